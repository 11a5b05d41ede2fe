// k_gemv_tile.hip — decode GEMV for 3..8 bf16 activation rows over the Q4_K /
// MLX affine tile plane, with exact (unrounded) weights.
//
// Role: the m = 2..8 projections of the reference (AffineQmpp,
// engine/src/quant_kernel.rs:3188-3738) over a second, tile-major copy of the
// weight, as the engine keeps its own tiled repack for those kernels
// (QLin::tiled, engine/src/qwen35.rs:629-697).  The row-quad plane stays the
// weight's primary copy (the M = 1 GEMV's contiguous 1-KB wave loads need it);
// thq_weight_add_tiles builds this one on the device.
//
// Why a second layout.  The MFMA decode GEMV on the row-quad plane gives each
// lane one weight row, so one wave load touches 64 cache lines in 16-B pieces
// (each line is finished by 8 later loads): the memory pipeline backs up and
// the stream runs at 0.25-0.3 of HBM.  In the tile plane (thq_dev.hpp,
// q4t_record) a 32-row tile's 64-weight part is 1 KB contiguous in exactly
// the MFMA B-operand order, so every wave load reads whole lines.
//
// Exactness, as in k_gemv_mfma: B = bf16(128 + q) from one v_perm per two
// nibbles, the MFMA gives A = sum x*(128 + q) per 32-weight sub-block, and
//   sum x*w = d1*A - (128*d1 + m1)*S         (Q4_K, d1 = d*sc, m1 = dmin*m)
//   sum x*w = s*A - (128*s - b)*S            (MLX affine, scale s, bias b)
// with S = sum x over the sub-block, taken while the rows are staged.
//
// Block: one 32-row output tile x KW waves over a K range of KW * 512
// columns.  Wave w owns two superblocks of the range: it loads rows x[0..M)
// of its 512 columns, issues all its weight loads (10 x 16 B per lane)
// behind them, stages its columns in LDS with their 32-wide sums (no block
// barrier: a wave reads only what it wrote), and accumulates its rows; the
// waves' partials are summed in LDS in wave order.  K beyond one block's range is
// split over blockIdx.y: f32 partials, summed in split order (deterministic)
// by the last block of each tile to arrive, or by k_split_reduce when the
// caller has no arrival counters.
#include "thq_dev.hpp"
#include "thq_kernels.hpp"

#include <algorithm>
#include <atomic>
#include <cstdlib>

namespace thq {
namespace {

constexpr int TL_CPB = 2;  // superblocks per wave
constexpr int TL_MX = 8;   // activation rows at most

// row-quad plane -> tile plane, one thread per 16-B chunk of the destination
__global__ __launch_bounds__(256) void k_repack_q4t(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                   int64_t n, int nsb, int64_t chunks) {
    const int64_t c = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (c >= chunks) return;
    const int64_t rec = c / 288;
    const int j = (int)(c % 288);
    const int64_t t = rec / nsb;
    const int s = (int)(rec % nsb);
    uint4 v = make_uint4(0, 0, 0, 0);
    if (j < 256) {
        const int64_t row = 32 * t + (j & 31);
        if (row < n) v = *reinterpret_cast<const uint4*>(src + q4k_piece(row, nsb, s, (j >> 5) & 1, j >> 6));
    } else {
        const int64_t row = 32 * t + (j - 256);
        if (row < n) {
            v.x = *reinterpret_cast<const uint32_t*>(src + q4k_hdword(row, nsb, s, 0));
            v.y = *reinterpret_cast<const uint32_t*>(src + q4k_hdword(row, nsb, s, 1));
            v.z = *reinterpret_cast<const uint32_t*>(src + q4k_hdword(row, nsb, s, 2));
            v.w = *reinterpret_cast<const uint32_t*>(src + q4k_hdword(row, nsb, s, 3));
        }
    }
    reinterpret_cast<uint4*>(dst)[c] = v;
}

__device__ __forceinline__ f32x16_t tmfma(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// low nibbles (masked to 4 bits) of the bytes of a, b -> bf16(128 + q) x 8 (exact)
__device__ __forceinline__ bf16x8_t tnib(uint32_t a, uint32_t b) {
    const uint32_t C = 0x43434343u;
    return as_bf16x8(make_uint4(__builtin_amdgcn_perm(C, a, 0x04010400u), __builtin_amdgcn_perm(C, a, 0x04030402u),
                                __builtin_amdgcn_perm(C, b, 0x04010400u), __builtin_amdgcn_perm(C, b, 0x04030402u)));
}
template <int CTRL>
__device__ __forceinline__ float tdpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

// LDS bytes of a block: x rows, 32-wide sums, the waves' partials (nt tiles)
constexpr size_t tile_lds_bytes(int kw, int m, int nt) {
    return (size_t)m * (kw * TL_CPB * 256 + 8) * 2 + (size_t)kw * TL_CPB * 8 * TL_MX * 4 +
           (size_t)(kw > 1 ? kw - 1 : 1) * nt * 4 * 64 * 4;
}

// The end of a tile block (both tile kernels): the waves' partials summed
// in LDS in wave order by wave 0, then y (silu(g)*u for gate/up) or, with
// SPLIT, the f32 partials and the split-order sum of the last block to arrive.
// tot[t][e]: weight row 32 tile + n of tile t, activation row 4g + e.
template <int KW, int NT, bool GU, typename YT, bool SPLIT>
__device__ __forceinline__ void tile_finish(float (&tot)[NT][4], float* red, YT* __restrict__ Y, float* __restrict__ P,
                                            uint32_t* __restrict__ cnt, int M, int64_t nout, int64_t tile, int wave,
                                            int lane) {
    const int n = lane & 31, g = lane >> 5;
    if constexpr (KW > 1) {
        if (wave > 0) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) red[(((wave - 1) * NT + t) * 4 + e) * 64 + lane] = tot[t][e];
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int k = 0; k < KW - 1; ++k)
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int e = 0; e < 4; ++e) tot[t][e] += red[((k * NT + t) * 4 + e) * 64 + lane];
        }
    }
    const int64_t row = tile * 32 + n;
    if constexpr (!SPLIT) {
        if (wave != 0 || row >= nout) return;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (4 * g + e < M)
                store_y<YT>(Y + (int64_t)(4 * g + e) * nout + row, GU ? silu_mul(tot[0][e], tot[NT - 1][e]) : tot[0][e]);
    } else {
        // partials as device-scope (sc1) stores when the last block sums them,
        // published before the ticket (ticket_publish, thq_dev.hpp) and read
        // back with device-scope loads after it
        const int64_t ldp = NT * nout;
        if (wave == 0 && row < nout) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int m = 4 * g + e;
                    if (m >= M) continue;
                    float* dst = P + ((int64_t)blockIdx.y * M + m) * ldp + t * nout + row;
                    if (cnt)
                        __hip_atomic_store(dst, tot[t][e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    else
                        *dst = tot[t][e];
                }
        }
        if (!cnt) return;
        __shared__ int last;
        ticket_publish();
        __syncthreads();
        if (threadIdx.x == 0) last = ticket_draw(cnt + tile) == gridDim.y - 1;
        __syncthreads();
        if (!last) return;
        // the tile's outputs, one per thread: the splits' partials in split
        // order (k_split_reduce's sums, bit for bit), loads batched 8 deep
        const int splits = (int)gridDim.y;
        for (int i = threadIdx.x; i < 32 * M; i += 64 * KW) {
            const int m = i >> 5;
            const int64_t r = tile * 32 + (i & 31);
            if (r >= nout) continue;
            float acc[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                acc[t] = 0.0f;
                for (int q0 = 0; q0 < splits; q0 += 8) {
                    float v[8];
#pragma unroll
                    for (int b = 0; b < 8; ++b)
                        v[b] = q0 + b < splits
                                   ? __hip_atomic_load(P + ((int64_t)(q0 + b) * M + m) * ldp + t * nout + r,
                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                   : 0.0f;
#pragma unroll
                    for (int b = 0; b < 8; ++b)
                        if (q0 + b < splits) acc[t] += v[b];
                }
            }
            store_y<YT>(Y + (int64_t)m * nout + r, GU ? silu_mul(acc[0], acc[NT - 1]) : acc[0]);
        }
        if (threadIdx.x == 0) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// K: x row stride (columns); nsb: superblocks in the plane (K padded to whole
// superblocks for MLX affine, whose padding groups are zero).  Plain: block
// x owns weight rows 32x .. 32x+31 = outputs, stored as y[m][nout].  Gate/up
// (GU, nout a multiple of 32): block x owns gate rows 32x .. and up rows
// nout + 32x .. of the [gate; up] weight, and stores silu(g)*u (the
// epilogue of every kernel, silu_mul) for outputs 32x ...  With SPLIT (K
// split over blockIdx.y) each block writes f32 partials P[blockIdx.y][m][ldp]
// (ldp = nout, or 2 nout with the up rows at nout + o); with arrival
// counters (cnt: one per output tile, zero before the launch and left zero)
// the last block of a tile to arrive sums them in split order into y, else
// k_split_reduce does.
template <int KW, bool AFF, bool GU, typename YT, bool SPLIT>
__global__ __launch_bounds__(64 * KW) void k_gemv_q4t(const uint8_t* __restrict__ T, const bf16_t* __restrict__ X,
                                                     YT* __restrict__ Y, float* __restrict__ P,
                                                     uint32_t* __restrict__ cnt, int M, int K, int nsb,
                                                     int64_t nout) {
    constexpr int NT = GU ? 2 : 1;         // weight tiles per block
    constexpr int KR = KW * TL_CPB * 256;  // the block's K range (columns)
    constexpr int XR = KR + 8;             // LDS row stride (bf16): rows start 16 B apart in bank order
    extern __shared__ __attribute__((aligned(16))) uint8_t tl_lds[];
    bf16_t* xs = reinterpret_cast<bf16_t*>(tl_lds);                // [M][XR]
    float* Ss = reinterpret_cast<float*>(tl_lds + (size_t)M * XR * 2);  // [KR / 32][TL_MX]
    float* red = Ss + (KR / 32) * TL_MX;                           // [KW - 1][NT][4][64]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 31, g = lane >> 5;
    const int64_t tile = blockIdx.x;
    const int sb0 = blockIdx.y * KW * TL_CPB;
    const int s0 = sb0 + wave * TL_CPB;

    // activation rows first (their loads drain before the weight loads):
    // each wave reads only its own 512 columns (lane: columns 8 lane ..
    // 8 lane + 7 of each row), so no block barrier stands before its math
    const int64_t col = (int64_t)s0 * 256 + 8 * lane;
    uint4 xv[TL_MX];
#pragma unroll
    for (int m = 0; m < TL_MX; ++m)
        if (m < M)
            xv[m] = col < K ? *reinterpret_cast<const uint4*>(X + (int64_t)m * K + col) : make_uint4(0, 0, 0, 0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    // the wave's weights: per tile and superblock the 32 rows' headers (lane
    // n) and the four 1-KB parts (lane (n, g): piece g of row n); superblocks
    // past the plane read the last one and count as zero
    uint4 hd[NT][TL_CPB], wq[NT][TL_CPB][4];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int64_t wt = tile + (t ? nout / 32 : 0);
#pragma unroll
        for (int c = 0; c < TL_CPB; ++c) {
            const int s = s0 + c < nsb ? s0 + c : nsb - 1;
            const uint8_t* rb = T + q4t_record(wt, nsb, s);
            hd[t][c] = *reinterpret_cast<const uint4*>(rb + 4096 + 16 * n);
#pragma unroll
            for (int p = 0; p < 4; ++p) wq[t][c][p] = *reinterpret_cast<const uint4*>(rb + p * 1024 + 16 * lane);
        }
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    // stage the wave's columns of the rows and their 32-wide sums (four
    // lanes per group); rows M .. TL_MX-1 of the sums are zero
    const int wc0 = wave * TL_CPB * 256;  // the wave's first column in the block's range
#pragma unroll
    for (int m = 0; m < TL_MX; ++m) {
        if (m < M) {
            const uint4 v = xv[m];
            *reinterpret_cast<uint4*>(xs + m * XR + wc0 + 8 * lane) = v;
            const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
            bf16x2_t q[4];
            __builtin_memcpy(q, &v, 16);
            float t = __builtin_amdgcn_fdot2_f32_bf16(q[0], one, 0.0f, false);
            t = __builtin_amdgcn_fdot2_f32_bf16(q[1], one, t, false);
            t = __builtin_amdgcn_fdot2_f32_bf16(q[2], one, t, false);
            t = __builtin_amdgcn_fdot2_f32_bf16(q[3], one, t, false);
            t = tdpp_add<0xB1>(t);  // quad_perm [1,0,3,2]
            t = tdpp_add<0x4E>(t);  // quad_perm [2,3,0,1]
            if ((lane & 3) == 0) Ss[((wc0 >> 5) + (lane >> 2)) * TL_MX + m] = t;
        } else if ((lane & 3) == 0) {
            Ss[((wc0 >> 5) + (lane >> 2)) * TL_MX + m] = 0.0f;
        }
    }
    // the wave reads back only what it wrote: its LDS operations complete in order
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();

    // A operand: lane (n, g) supplies activation row n (rows >= M are zero);
    // the output lane holds weight row n and activation rows 4g + e, e < 4
    const bool arow = n < M;
    const bf16_t* xa = xs + (arow ? n : 0) * XR + 16 * g + wave * TL_CPB * 256;
    const int sbase = wave * TL_CPB * 8;
    const f32x16_t z16 = {};
    float tot[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) tot[t][e] = 0.0f;
    const uint32_t M4 = 0x0F0F0F0Fu;
#pragma unroll
    for (int c = 0; c < TL_CPB; ++c) {
        const bool live = s0 + c < nsb;
        float d[NT], dm[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            d[t] = (!AFF && live) ? q4k_hdr_d(hd[t][c]) : 0.0f;
            dm[t] = (!AFF && live) ? q4k_hdr_dmin(hd[t][c]) : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int kl = c * 256 + u * 64;
            uint4 a0 = {}, a1 = {}, a2 = {}, a3 = {};
            if (arow) {
                a0 = *reinterpret_cast<const uint4*>(xa + kl);
                a1 = *reinterpret_cast<const uint4*>(xa + kl + 8);
                a2 = *reinterpret_cast<const uint4*>(xa + kl + 32);
                a3 = *reinterpret_cast<const uint4*>(xa + kl + 40);
            }
            const f32x4_t S1 = *reinterpret_cast<const f32x4_t*>(&Ss[(sbase + (kl >> 5)) * TL_MX + 4 * g]);
            const f32x4_t S2 = *reinterpret_cast<const f32x4_t*>(&Ss[(sbase + (kl >> 5) + 1) * TL_MX + 4 * g]);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const uint4 hh = hd[t][c];
                const uint32_t hw = u == 0 ? hh.x : (u == 1 ? hh.y : (u == 2 ? hh.z : hh.w));
                float d1, d2, c1, c2;
                if constexpr (AFF) {  // one 64-weight group: w = s*q + b = s*(128 + q) - (128*s - b)
                    const float sc = live ? aff_scale(hw) : 0.0f, bi = live ? aff_bias(hw) : 0.0f;
                    d1 = d2 = sc;
                    c1 = c2 = __builtin_fmaf(128.0f, sc, -bi);
                } else {
                    d1 = d[t] * (float)(hw & 63u);
                    d2 = d[t] * (float)((hw >> 12) & 63u);
                    c1 = __builtin_fmaf(128.0f, d1, dm[t] * (float)((hw >> 6) & 63u));
                    c2 = __builtin_fmaf(128.0f, d2, dm[t] * (float)((hw >> 18) & 63u));
                }
                const uint4 q = wq[t][c][u];
                f32x16_t A = tmfma(as_bf16x8(a0), tnib(q.x & M4, q.y & M4), z16);
                f32x16_t B = tmfma(as_bf16x8(a2), tnib((q.x >> 4) & M4, (q.y >> 4) & M4), z16);
                A = tmfma(as_bf16x8(a1), tnib(q.z & M4, q.w & M4), A);
                B = tmfma(as_bf16x8(a3), tnib((q.z >> 4) & M4, (q.w >> 4) & M4), B);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    tot[t][e] = __builtin_fmaf(-c1, S1[e], __builtin_fmaf(d1, A[e], tot[t][e]));
                    tot[t][e] = __builtin_fmaf(-c2, S2[e], __builtin_fmaf(d2, B[e], tot[t][e]));
                }
                // one part at a time: left free, the compiler issues every
                // part's MFMAs first and keeps all their results live
#pragma unroll
                for (int e = 0; e < 4; ++e) asm volatile("" : "+v"(tot[t][e]));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    tile_finish<KW, NT, GU, YT, SPLIT>(tot, red, Y, P, cnt, M, nout, tile, wave, lane);
}

typedef int ti32x4 __attribute__((ext_vector_type(4)));
typedef int ti32x16 __attribute__((ext_vector_type(16)));

// LDS bytes of a THQ_MODE_Q8ACT tile block: int8 x rows, the 32-quant sums,
// the rows' Q8_K d, the waves' partials (nt tiles)
constexpr size_t q8t_lds_bytes(int kw, int m, int nt) {
    return (size_t)m * (kw * TL_CPB * 256 + 32) + (size_t)kw * TL_CPB * 8 * TL_MX * 4 +
           (size_t)kw * TL_CPB * TL_MX * 4 + (size_t)(kw > 1 ? kw - 1 : 1) * nt * 4 * 64 * 4;
}

// THQ_MODE_Q8ACT (candle's k_quants::matmul: Q4_K weights against Q8_K
// activations, [ext] BlockQ4K::vec_dot) over the tile plane, 1..8 rows.
// Same block and wave structure as k_gemv_q4t; the activation operand is the
// Q8_K planes (xq [M][K] i8, xd [M][K/256] f32 d, xb [M][K/32] i16 sums of
// 32 quants).  Per 32-weight sub-block j one v_mfma_i32_32x32x32_i8 forms
// every (activation row, weight row) integer (q4 . q8)_j exactly: B = the
// tile piece's low (sub-block 2p) or high (2p + 1) nibbles as they lie in
// the loaded 16 B, A = the activation row's 16 quants of the same half.  Per
// superblock and output the integers
//   aux = sum_j sc_j * (q4 . q8)_j,   mins = sum_j m_j * xb_j
// enter the total as (d_w * d_x) * aux - (dmin_w * d_x) * mins, the f32 step
// of k_q8act_q4k.
template <int KW, bool GU, typename YT, bool SPLIT>
__global__ __launch_bounds__(64 * KW) void k_q8act_q4t(const uint8_t* __restrict__ T, const int8_t* __restrict__ XQ,
                                                      const float* __restrict__ XD, const int16_t* __restrict__ XB,
                                                      YT* __restrict__ Y, float* __restrict__ P,
                                                      uint32_t* __restrict__ cnt, int M, int nsb, int64_t nout) {
    constexpr int NT = GU ? 2 : 1;
    constexpr int KR = KW * TL_CPB * 256;  // the block's K range (columns)
    constexpr int XR = KR + 32;            // LDS row stride (bytes): rows start 32 B apart in bank order
    extern __shared__ __attribute__((aligned(16))) uint8_t tl_lds[];
    int8_t* xs = reinterpret_cast<int8_t*>(tl_lds);                  // [M][XR]
    int* Sb = reinterpret_cast<int*>(tl_lds + (size_t)M * XR);        // [KR / 32][TL_MX]
    float* Dx = reinterpret_cast<float*>(Sb + (KR / 32) * TL_MX);     // [KW * TL_CPB][TL_MX]
    float* red = Dx + KW * TL_CPB * TL_MX;                            // [KW - 1][NT][4][64]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 31, g = lane >> 5;
    const int64_t tile = blockIdx.x;
    const int s0 = blockIdx.y * KW * TL_CPB + wave * TL_CPB;
    const int64_t K = (int64_t)nsb * 256;
    const int nsub = nsb * 8;

    // the wave's activation data first: 8 quants per lane and row; the
    // sums of its 16 sub-blocks (lane: row lane / 8, sub-blocks 2 (lane % 8)
    // and + 1); d of its two superblocks (lanes 0..15: row lane / 2)
    const int64_t col = (int64_t)s0 * 256 + 8 * lane;
    uint2 xv[TL_MX];
#pragma unroll
    for (int m = 0; m < TL_MX; ++m)
        if (m < M) xv[m] = col < K ? *reinterpret_cast<const uint2*>(XQ + m * K + col) : make_uint2(0, 0);
    const int mb = lane >> 3, j2 = lane & 7;
    const int sub = s0 * 8 + 2 * j2;
    uint32_t bs = 0;
    if (mb < M && sub < nsub) bs = *reinterpret_cast<const uint32_t*>(XB + (int64_t)mb * nsub + sub);
    const int md = (lane >> 1) & (TL_MX - 1), cd = lane & 1;
    float dxv = 0.0f;
    if (lane < 2 * TL_MX && md < M && s0 + cd < nsb) dxv = XD[(int64_t)md * nsb + s0 + cd];
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    // the wave's weights, as in k_gemv_q4t
    uint4 hd[NT][TL_CPB], wq[NT][TL_CPB][4];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int64_t wt = tile + (t ? nout / 32 : 0);
#pragma unroll
        for (int c = 0; c < TL_CPB; ++c) {
            const int s = s0 + c < nsb ? s0 + c : nsb - 1;
            const uint8_t* rb = T + q4t_record(wt, nsb, s);
            hd[t][c] = *reinterpret_cast<const uint4*>(rb + 4096 + 16 * n);
#pragma unroll
            for (int p = 0; p < 4; ++p) wq[t][c][p] = *reinterpret_cast<const uint4*>(rb + p * 1024 + 16 * lane);
        }
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    // stage (rows M .. TL_MX-1 of the sums and d are zero); the wave reads
    // back only what it wrote
    const int wc0 = wave * TL_CPB * 256;
#pragma unroll
    for (int m = 0; m < TL_MX; ++m)
        if (m < M) *reinterpret_cast<uint2*>(xs + m * XR + wc0 + 8 * lane) = xv[m];
    Sb[((wc0 >> 5) + 2 * j2) * TL_MX + mb] = (int)(int16_t)(bs & 0xFFFFu);
    Sb[((wc0 >> 5) + 2 * j2 + 1) * TL_MX + mb] = (int)(int16_t)(bs >> 16);
    if (lane < 2 * TL_MX) Dx[(wave * TL_CPB + cd) * TL_MX + md] = dxv;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();

    // A operand: lane (n, g) supplies activation row n (rows >= M are zero);
    // the output lane holds weight row n and activation rows 4g + e, e < 4
    const bool arow = n < M;
    const int8_t* xa = xs + (arow ? n : 0) * XR + 16 * g + wc0;
    const ti32x16 z16 = {};
    const uint32_t M4 = 0x0F0F0F0Fu;
    float tot[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) tot[t][e] = 0.0f;
#pragma unroll
    for (int c = 0; c < TL_CPB; ++c) {
        int aux[NT][4], mns[NT][4];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) aux[t][e] = mns[t][e] = 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int kl = c * 256 + u * 64;
            ti32x4 a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
            if (arow) {
                a0 = *reinterpret_cast<const ti32x4*>(xa + kl);
                a1 = *reinterpret_cast<const ti32x4*>(xa + kl + 32);
            }
            const int jb = (wc0 >> 5) + (kl >> 5);
            const ti32x4 b0 = *reinterpret_cast<const ti32x4*>(&Sb[jb * TL_MX + 4 * g]);
            const ti32x4 b1 = *reinterpret_cast<const ti32x4*>(&Sb[(jb + 1) * TL_MX + 4 * g]);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const uint4 hh = hd[t][c];
                const uint32_t hw = u == 0 ? hh.x : (u == 1 ? hh.y : (u == 2 ? hh.z : hh.w));
                const uint4 q = wq[t][c][u];
                const ti32x4 lo = {(int)(q.x & M4), (int)(q.y & M4), (int)(q.z & M4), (int)(q.w & M4)};
                const ti32x4 hi = {(int)((q.x >> 4) & M4), (int)((q.y >> 4) & M4), (int)((q.z >> 4) & M4),
                                   (int)((q.w >> 4) & M4)};
                const ti32x16 C0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, lo, z16, 0, 0, 0);
                const ti32x16 C1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, hi, z16, 0, 0, 0);
                const int sc0 = (int)(hw & 63u), mn0 = (int)((hw >> 6) & 63u);
                const int sc1 = (int)((hw >> 12) & 63u), mn1 = (int)((hw >> 18) & 63u);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    aux[t][e] += __mul24(sc0, C0[e]) + __mul24(sc1, C1[e]);
                    mns[t][e] += __mul24(mn0, b0[e]) + __mul24(mn1, b1[e]);
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) asm volatile("" : "+v"(aux[t][e]), "+v"(mns[t][e]));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (s0 + c < nsb) {
            const f32x4_t dx = *reinterpret_cast<const f32x4_t*>(&Dx[(wave * TL_CPB + c) * TL_MX + 4 * g]);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float dw = q4k_hdr_d(hd[t][c]), dmw = q4k_hdr_dmin(hd[t][c]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float dd = dw * dx[e], dm = dmw * dx[e];
                    tot[t][e] = __builtin_fmaf(-dm, (float)mns[t][e], __builtin_fmaf(dd, (float)aux[t][e], tot[t][e]));
                }
            }
        }
    }
    tile_finish<KW, NT, GU, YT, SPLIT>(tot, red, Y, P, cnt, M, nout, tile, wave, lane);
}

template <int KW, bool AFF, bool GU, typename YT>
hipError_t launch_kwy(const TilePlan& p, const uint8_t* T, const bf16_t* x, YT* y, int M, int K, int nsb,
                      int64_t nout, float* ws, uint32_t* cnt, hipStream_t s) {
    const dim3 grid((unsigned)((nout + 31) / 32), (unsigned)p.splits);
    const size_t lds = tile_lds_bytes(KW, M, GU ? 2 : 1);
    if (p.splits == 1) {
        hipLaunchKernelGGL((k_gemv_q4t<KW, AFF, GU, YT, false>), grid, dim3(64 * KW), lds, s, T, x, y,
                           (float*)nullptr, (uint32_t*)nullptr, M, K, nsb, nout);
        return hipGetLastError();
    }
    hipLaunchKernelGGL((k_gemv_q4t<KW, AFF, GU, YT, true>), grid, dim3(64 * KW), lds, s, T, x, y, ws, cnt, M, K, nsb,
                       nout);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || cnt) return e;
    return launch_split_reduce(ws, y, sizeof(YT) == 4, GU, M, nout, GU ? nout : 0, GU ? 2 * nout : nout, p.splits,
                               s);
}

template <int KW, bool AFF, bool GU>
hipError_t launch_kw(const TilePlan& p, const uint8_t* T, const void* x, void* y, bool yf32, int M, int K, int nsb,
                     int64_t nout, float* ws, uint32_t* cnt, hipStream_t s) {
    // more than 64 KB of dynamic LDS (8 rows, 8 waves) must be allowed per
    // kernel and device, once
    constexpr size_t lds_max = tile_lds_bytes(KW, TL_MX, GU ? 2 : 1);
    if constexpr (lds_max > 65536) {
        static std::atomic<uint64_t> allowed{0};
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) dev = 0;
        const uint64_t bit = 1ull << (dev & 63);
        if (!(allowed.load() & bit)) {
            const void* fns[4] = {(const void*)k_gemv_q4t<KW, AFF, GU, float, true>,
                                  (const void*)k_gemv_q4t<KW, AFF, GU, float, false>,
                                  (const void*)k_gemv_q4t<KW, AFF, GU, bf16_t, true>,
                                  (const void*)k_gemv_q4t<KW, AFF, GU, bf16_t, false>};
            for (const void* f : fns) {
                const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_max);
                if (e != hipSuccess) return e;
            }
            allowed.fetch_or(bit);
        }
    }
    const bf16_t* xb = static_cast<const bf16_t*>(x);
    if (yf32) return launch_kwy<KW, AFF, GU, float>(p, T, xb, static_cast<float*>(y), M, K, nsb, nout, ws, cnt, s);
    return launch_kwy<KW, AFF, GU, bf16_t>(p, T, xb, static_cast<bf16_t*>(y), M, K, nsb, nout, ws, cnt, s);
}

template <bool AFF, bool GU>
hipError_t launch_t(const TilePlan& p, const uint8_t* T, const void* x, void* y, bool yf32, int M, int K, int nsb,
                    int64_t nout, float* ws, uint32_t* cnt, hipStream_t s) {
    switch (p.kw) {
        case 8: return launch_kw<8, AFF, GU>(p, T, x, y, yf32, M, K, nsb, nout, ws, cnt, s);
        case 4: return launch_kw<4, AFF, GU>(p, T, x, y, yf32, M, K, nsb, nout, ws, cnt, s);
        case 2: return launch_kw<2, AFF, GU>(p, T, x, y, yf32, M, K, nsb, nout, ws, cnt, s);
        default: return launch_kw<1, AFF, GU>(p, T, x, y, yf32, M, K, nsb, nout, ws, cnt, s);
    }
}

template <int KW, bool GU, typename YT>
hipError_t launch_q8t_kwy(const TilePlan& p, const uint8_t* T, const int8_t* xq, const float* xd, const int16_t* xb,
                          YT* y, int M, int nsb, int64_t nout, float* ws, uint32_t* cnt, hipStream_t s) {
    static_assert(q8t_lds_bytes(KW, TL_MX, GU ? 2 : 1) <= 65536, "Q8ACT tile block beyond 64 KB of LDS");
    const dim3 grid((unsigned)((nout + 31) / 32), (unsigned)p.splits);
    const size_t lds = q8t_lds_bytes(KW, M, GU ? 2 : 1);
    if (p.splits == 1) {
        hipLaunchKernelGGL((k_q8act_q4t<KW, GU, YT, false>), grid, dim3(64 * KW), lds, s, T, xq, xd, xb, y,
                           (float*)nullptr, (uint32_t*)nullptr, M, nsb, nout);
        return hipGetLastError();
    }
    hipLaunchKernelGGL((k_q8act_q4t<KW, GU, YT, true>), grid, dim3(64 * KW), lds, s, T, xq, xd, xb, y, ws, cnt, M,
                       nsb, nout);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || cnt) return e;
    return launch_split_reduce(ws, y, sizeof(YT) == 4, GU, M, nout, GU ? nout : 0, GU ? 2 * nout : nout, p.splits,
                               s);
}

template <bool GU, typename YT>
hipError_t launch_q8t(const TilePlan& p, const uint8_t* T, const int8_t* xq, const float* xd, const int16_t* xb, YT* y,
                      int M, int nsb, int64_t nout, float* ws, uint32_t* cnt, hipStream_t s) {
    switch (p.kw) {
        case 8: return launch_q8t_kwy<8, GU, YT>(p, T, xq, xd, xb, y, M, nsb, nout, ws, cnt, s);
        case 4: return launch_q8t_kwy<4, GU, YT>(p, T, xq, xd, xb, y, M, nsb, nout, ws, cnt, s);
        case 2: return launch_q8t_kwy<2, GU, YT>(p, T, xq, xd, xb, y, M, nsb, nout, ws, cnt, s);
        default: return launch_q8t_kwy<1, GU, YT>(p, T, xq, xd, xb, y, M, nsb, nout, ws, cnt, s);
    }
}

}  // namespace

size_t tile_plane_bytes(int64_t n, int64_t k) { return (size_t)q4t_bytes(n, (int)((k + 255) / 256)); }

hipError_t launch_repack_q4t(const uint8_t* rowquad, uint8_t* tiles, int64_t n, int64_t k, hipStream_t s) {
    const int nsb = (int)((k + 255) / 256);
    const int64_t chunks = (n + 31) / 32 * nsb * 288;
    hipLaunchKernelGGL(k_repack_q4t, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, s, rowquad, tiles, n, nsb,
                       chunks);
    return hipGetLastError();
}

// Waves per block and K splits: the largest block (8 waves, 4096 columns)
// whose grid still holds one block per CU, 4 waves when K needs splits
// anyway; more splits only when the tiles alone cannot fill the GPU.
// Gate/up: nout = N / 2 outputs (a multiple of 32), partials of both halves.
TilePlan plan_gemv_tile(int64_t M, int64_t N, int64_t K, bool gu, int cus) {
    TilePlan p;
    if (M < 1 || M > TL_MX || N < 1 || K < 256) return p;
    if (gu && (N % 64)) return p;
    if (cus < 1) cus = 256;
    const int nsb = (int)((K + 255) / 256);
    const int64_t nout = gu ? N / 2 : N;
    const int64_t tiles = (nout + 31) / 32;
    int kw = 8;
    while (kw > 1 && tiles * ((nsb + kw * TL_CPB - 1) / (kw * TL_CPB)) < cus) kw >>= 1;
    // never more waves than superblock pairs in K
    while (kw > 1 && (kw / 2) * TL_CPB >= nsb) kw >>= 1;
    // a K that needs splits anyway: 4-wave blocks, which spread over the CUs
    // evenly (4096 x 12288, M = 3..8: 6 splits 11.0-11.9 us against 3 splits
    // of 8-wave blocks 12.0-13.3 us; 12288 x 4096 keeps one split of 8 waves,
    // 10.4-11.4 us against 10.8-11.7)
    if (kw == 8 && nsb > 8 * TL_CPB) kw = 4;
    // gate/up holds both tiles' weights (156 VGPRs, 3 waves per SIMD): one
    // 8-wave block per CU would leave a third of the slots idle, three
    // 4-wave blocks fill them
    if (gu && kw == 8) kw = 4;
    // tuning override: THQ_TILE_KW = 1, 2, 4 or 8 waves per block
    if (const char* e = getenv("THQ_TILE_KW")) {
        const int v = atoi(e);
        if (v == 1 || v == 2 || v == 4 || v == 8) kw = v;
    }
    p.kw = kw;
    p.splits = (nsb + kw * TL_CPB - 1) / (kw * TL_CPB);
    p.workspace_bytes = p.splits > 1 ? (size_t)p.splits * (size_t)M * (size_t)N * sizeof(float) : 0;
    return p;
}

hipError_t launch_gemv_tile(const TilePlan& p, const WeightView& w, const uint8_t* tiles, const void* x, void* y,
                            bool yf32, bool gu, int M, float* ws, uint32_t* cnt, hipStream_t s) {
    if (p.kw == 0 || (w.qtype != 12 && w.qtype != 13) || (gu && (w.N % 64))) return hipErrorInvalidValue;
    const int nsb = (int)((w.K + 255) / 256);
    const int64_t nout = gu ? w.N / 2 : w.N;
    if (w.qtype == 13)
        return gu ? launch_t<true, true>(p, tiles, x, y, yf32, M, (int)w.K, nsb, nout, ws, cnt, s)
                  : launch_t<true, false>(p, tiles, x, y, yf32, M, (int)w.K, nsb, nout, ws, cnt, s);
    return gu ? launch_t<false, true>(p, tiles, x, y, yf32, M, (int)w.K, nsb, nout, ws, cnt, s)
              : launch_t<false, false>(p, tiles, x, y, yf32, M, (int)w.K, nsb, nout, ws, cnt, s);
}

hipError_t launch_q8act_tile(const TilePlan& p, const WeightView& w, const uint8_t* tiles, const int8_t* xq,
                             const float* xd, const int16_t* xb, void* y, bool yf32, bool gu, int M, float* ws,
                             uint32_t* cnt, hipStream_t s) {
    if (p.kw == 0 || w.qtype != 12 || w.K % 256 || M < 1 || M > TL_MX || (gu && (w.N % 64)))
        return hipErrorInvalidValue;
    const int nsb = (int)(w.K / 256);
    const int64_t nout = gu ? w.N / 2 : w.N;
    if (yf32)
        return gu ? launch_q8t<true, float>(p, tiles, xq, xd, xb, static_cast<float*>(y), M, nsb, nout, ws, cnt, s)
                  : launch_q8t<false, float>(p, tiles, xq, xd, xb, static_cast<float*>(y), M, nsb, nout, ws, cnt, s);
    return gu ? launch_q8t<true, bf16_t>(p, tiles, xq, xd, xb, static_cast<bf16_t*>(y), M, nsb, nout, ws, cnt, s)
              : launch_q8t<false, bf16_t>(p, tiles, xq, xd, xb, static_cast<bf16_t*>(y), M, nsb, nout, ws, cnt, s);
}

}  // namespace thq
