// k_gemm_mid.hip — prefill / verify GEMM for tens to hundreds of bf16
// activation rows over Q4_K / MLX affine weights in the default row-quad
// layout, with rounded weights.
//
// Role: the middle of the reference's prefill range (pf_policy,
// engine/src/quant_kernel.rs:5254-5300: the prefill GEMM over 4-bit
// weights; prefill steps of 512 rows, engine/src/main.rs:75-78), where the
// M x N output is too small for 256-wide GEMM tiles to fill the GPU without
// splitting K several ways.
//
// Structure (a block = NW waves, 4 or 8; its instances and the planner are
// below):
//   weights      each wave owns NT 32-row column tiles of weight rows
//                (gate/up: 16 gate rows and the 16 up rows of the same
//                outputs per tile); each lane streams its rows' 16-B nibble
//                pieces and header dwords of a 256-wide chunk straight into
//                registers (k_gemv_wide's loads), two chunks ahead of the
//                math, so every weight byte is read once per group of
//                activation rows;
//   activations  a group of up to MP = 32 MH rows is copied chunk by chunk
//                into LDS by direct-to-LDS copies (global_load_lds_dwordx4),
//                the next chunk while the current one computes: two buffers
//                of MP x 256 bf16.  One copy instruction fills two 512-B
//                rows; the 16-B piece p of row r sits at slot p ^ (r & 15),
//                so the MFMA operand reads of 16 consecutive rows hit 16
//                distinct bank groups.  Rows past M copy row M - 1 and are
//                never stored;
//   math         per 64-wide unit the lane's 32 weights per tile become bf16
//                fma(d1, 128 + q, -(128 d1 + m1)) (k_gemm's rounded tile,
//                bit for bit: Q4_K d1 = d sc, m1 = dmin m; affine d1 = scale,
//                m1 = -bias) and feed one v_mfma_f32_32x32x16_bf16 per 16 K
//                per 32-row half of the group and tile, accumulating across
//                all of K (no per-sub-block scaling);
//   K splits     f32 partials into the workspace, summed in split order by
//                k_split_reduce (deterministic).
// Offsets are 32-bit: the host checks the plane and x sizes (< 4 GiB).
#include "thq_dev.hpp"
#include "thq_kernels.hpp"
#include "thq_wave.hpp"

#include <cstdlib>
#include <cstring>
#include <type_traits>

namespace thq {
namespace {

constexpr int GM_KC = 256;              // K chunk (one superblock)

__device__ __forceinline__ uint32_t gm_lds(const void* p) {
    return (uint32_t)(size_t)(__attribute__((address_space(3))) const void*)p;
}
// lane l's 16 bytes at base + voff land at LDS m0 + 16 l; untracked by the
// compiler (the kernel waits for them itself)
__device__ __forceinline__ void gm_dma16(uint32_t lds, const void* base, uint32_t voff) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"{m0}"(lds), "v"(voff), "s"(base) : "memory");
}
template <int N>
__device__ __forceinline__ void gm_vmwait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ f32x16_t gm_mfma(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// 4 + 4 nibbles (bytes of a, then of b, bits 0..3) -> bf16 fma(s, 128 + q, -c) x 8
__device__ __forceinline__ bf16x8_t gm_deq(uint32_t a, uint32_t b, float s, float c) {
    const uint32_t E = 0x43434343u;
    auto f = [&](uint32_t v, int i) {
        return __builtin_fmaf(s, __uint_as_float(__builtin_amdgcn_perm(E, v, 0x04000c0cu | ((uint32_t)i << 16))), -c);
    };
    return as_bf16x8(make_uint4(pack_bf16x2(f(a, 0), f(a, 1)), pack_bf16x2(f(a, 2), f(a, 3)),
                                pack_bf16x2(f(b, 0), f(b, 1)), pack_bf16x2(f(b, 2), f(b, 3))));
}

// one 256-wide chunk of a lane's NT weight rows: 4 nibble pieces and 4
// header dwords each (8 NT load instructions)
typedef uint32_t gm_u32x4 __attribute__((ext_vector_type(4)));
template <int NT>
struct GmChunk {
    gm_u32x4 w[NT][4];
    uint32_t s[NT][4];
};
// the chunk's registers count as written here: the compiler waits for their
// loads at this point and keeps no copies across it
template <int NT>
__device__ __forceinline__ void gm_settle(GmChunk<NT>& C) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        asm volatile("" : "+v"(C.w[t][0]), "+v"(C.w[t][1]), "+v"(C.w[t][2]), "+v"(C.w[t][3])::"memory");
        asm volatile("" : "+v"(C.s[t][0]), "+v"(C.s[t][1]), "+v"(C.s[t][2]), "+v"(C.s[t][3])::"memory");
    }
}

// Blocks: (weight tile of 32 NW NT rows (gate/up: 16 NW NT outputs), K
// split, activation group of MP = 32 MH rows); NW waves (4, or 8: two per
// SIMD, so that one wave's weight conversion runs beside the other's
// MFMAs), each owning NT 32-row column tiles of the MFMA (one A operand
// read from LDS feeds NT MFMAs).
// The grid is one-dimensional and blocks are dealt round-robin to the 8
// XCDs: block b is renumbered so that each XCD runs a contiguous range of
// (split, group) keys with the weight tiles fastest, so an XCD copies the
// activations of one or two keys and keeps them in its own L2.
template <int QT, int MH, int NT, int NW, bool GU, bool SPLIT, typename YT>
__global__ __launch_bounds__(64 * NW, NW == 4 && MH * NT <= 2 ? 2 : 1) void k_gemm_mid(const uint8_t* Wq, const bf16_t* X,
                                                                      void* __restrict__ Yv, int M, int K,
                                                                      int64_t nout, int64_t up_off, int64_t nrows,
                                                                      int cps, int tiles, int splits) {
    constexpr int MP = 32 * MH;               // activation rows per group
    constexpr int XB = MP * 512;              // bytes per activation buffer
    constexpr int NJ = MP / (2 * NW);         // copy instructions per wave per chunk
    constexpr int WLOADS = 8 * NT;            // weight load instructions per chunk
    __shared__ __attribute__((aligned(16))) uint8_t xs[2 * XB];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 31, g = lane >> 5;
    int tile_i, split, group;
    {
        const int nb = gridDim.x, b = blockIdx.x;
        const int q = (nb + 7) >> 3, tall = (nb & 7) ? (nb & 7) : 8;  // XCDs 0 .. tall-1 run q blocks, the rest q - 1
        const int xcd = b & 7, local = b >> 3;
        const int v = xcd < tall ? xcd * q + local : tall * q + (xcd - tall) * (q - 1) + local;
        tile_i = v % tiles;
        split = (v / tiles) % splits;
        group = v / (tiles * splits);
    }
    const int64_t tile = tile_i;
    const int nch = K >> 8;
    const int cb = split * cps;
    const int ce = cb + cps < nch ? cb + cps : nch;
    const int m0 = group * MP;
    const int Mz = M - m0 < MP ? M - m0 : MP;  // rows of this group

    // column tile t of the wave: output orow[t]; weight row row[t]
    // (gate/up: lanes n < 16 the gate row, n >= 16 the up row of one output)
    const int nsb = K >> 8;
    int64_t orow[NT], row[NT];
    bool valid[NT];
    uint32_t ow[NT], os[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        orow[t] = GU ? tile * (16 * NW * NT) + (wave * NT + t) * 16 + (n & 15)
                     : tile * (32 * NW * NT) + (wave * NT + t) * 32 + n;
        valid[t] = orow[t] < nout;
        row[t] = GU && n >= 16 ? orow[t] + up_off : orow[t];
        if (!valid[t]) row[t] = 0;  // in-bounds reads; its weights convert to zero
        ow[t] = (uint32_t)q4k_piece(row[t], nsb, 0, g, 0);
        os[t] = (uint32_t)q4k_hdword(row[t], nsb, 0, 0);
    }
    auto wload = [&](GmChunk<NT>& C, int c) {
        const uint8_t* wc = Wq + (int64_t)c * 64;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                C.w[t][u] = *reinterpret_cast<const gm_u32x4*>(wc + ow[t] + u * 16);
                C.s[t][u] = *reinterpret_cast<const uint32_t*>(wc + os[t] + u * 16);
            }
    };

    // copy j of a wave fills rows 2 (wave + NW j) and 2 (wave + NW j) + 1;
    // lane l: row 2 (wave + NW j) + l / 32, LDS slot l % 32 <- piece (l % 32) ^ (row & 15)
    const uint32_t K2 = (uint32_t)K * 2u;
    uint32_t xoff[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int r = 2 * (wave + NW * j) + (lane >> 5);
        const int rr = r < Mz ? r : Mz - 1;
        xoff[j] = (uint32_t)(m0 + rr) * K2 + 16u * (uint32_t)((lane & 31) ^ (r & 15));
    }
    const uint32_t xs0 = gm_lds(xs);
    auto xcopy = [&](int c, int b) {
        const uint8_t* xc = reinterpret_cast<const uint8_t*>(X) + (int64_t)c * (GM_KC * 2);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
            gm_dma16(__builtin_amdgcn_readfirstlane(xs0 + (uint32_t)(b * XB + (wave + NW * j) * 1024)), xc,
                     xoff[j]);
    };
    // A operand of half h, unit u, part k (columns 16 g + 64 u + {0, 8, 32, 40}):
    // piece 2 g + 8 u + {0, 1, 4, 5} of row 32 h + n
    auto aread = [&](const uint8_t* xb, int h, int u, int k) {
        const int p = 2 * g + 8 * u + (k & 1) + 4 * (k >> 1);
        const uint8_t* a = xb + (32 * h + n) * 512 + 16 * (p ^ (n & 15));
        return as_bf16x8(*reinterpret_cast<const uint4*>(a));
    };

    f32x16_t acc[NT][MH];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int h = 0; h < MH; ++h) acc[t][h] = f32x16_t{};

    // Chunk math, software-pipelined by one 16-wide K step: step (u, k)
    // issues the A operand reads of the next step, then its own MFMAs, then
    // the conversion of one quarter of the next unit's weights (VALU that
    // runs while the MFMAs do), so no MFMA waits on a just-issued LDS read.
    auto compute = [&](const GmChunk<NT>& C, int b) {
        const uint8_t* xb = xs + b * XB;
        float d[NT], dm[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            d[t] = dm[t] = 0.0f;
            if constexpr (QT == 12) {
                d[t] = f16_to_f32((uint16_t)__builtin_amdgcn_perm(C.s[t][1], C.s[t][0], 0x0c0c0703u));
                dm[t] = f16_to_f32((uint16_t)__builtin_amdgcn_perm(C.s[t][3], C.s[t][2], 0x0c0c0703u));
                if (!valid[t]) d[t] = dm[t] = 0.0f;
            }
        }
        // unit u's scale and offset of tile t: [0], [1] low nibbles (sub-block
        // 2u), [2], [3] high nibbles (2u + 1)
        auto scales = [&](int t, int u, float (&sc)[4]) {
            const uint32_t hw = C.s[t][u];
            if constexpr (QT == 13) {
                const float a = valid[t] ? aff_scale(hw) : 0.0f, bi = valid[t] ? aff_bias(hw) : 0.0f;
                sc[0] = sc[2] = a;
                sc[1] = sc[3] = __builtin_fmaf(128.0f, a, -bi);
            } else {
                sc[0] = d[t] * (float)(hw & 63u);
                sc[1] = __builtin_fmaf(128.0f, sc[0], dm[t] * (float)((hw >> 6) & 63u));
                sc[2] = d[t] * (float)((hw >> 12) & 63u);
                sc[3] = __builtin_fmaf(128.0f, sc[2], dm[t] * (float)((hw >> 18) & 63u));
            }
        };
        const uint32_t M4 = 0x0F0F0F0Fu;
        // quarter k of unit u of tile t: 8 weights of the MFMA's 16-wide K step k
        auto conv = [&](int t, int u, int k, const float (&sc)[4]) {
            const gm_u32x4 q = C.w[t][u];
            const uint32_t a = k & 1 ? q.z : q.x, bb = k & 1 ? q.w : q.y;
            return k < 2 ? gm_deq(a & M4, bb & M4, sc[0], sc[1]) : gm_deq((a >> 4) & M4, (bb >> 4) & M4, sc[2], sc[3]);
        };
        bf16x8_t Bc[NT][4], Bn[NT][4];
        float sc[NT][4];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            scales(t, 0, sc[t]);
#pragma unroll
            for (int k = 0; k < 4; ++k) Bc[t][k] = conv(t, 0, k, sc[t]);
        }
        bf16x8_t Ac[MH], An[MH];
#pragma unroll
        for (int h = 0; h < MH; ++h) Ac[h] = aread(xb, h, 0, 0);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (u < 3) {
#pragma unroll
                for (int t = 0; t < NT; ++t) scales(t, u + 1, sc[t]);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int un = k == 3 ? u + 1 : u, kn = (k + 1) & 3;
                if (un < 4) {
#pragma unroll
                    for (int h = 0; h < MH; ++h) An[h] = aread(xb, h, un, kn);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int h = 0; h < MH; ++h)
#pragma unroll
                    for (int t = 0; t < NT; ++t) acc[t][h] = gm_mfma(Ac[h], Bc[t][k], acc[t][h]);
                __builtin_amdgcn_sched_barrier(0);
                if (u < 3) {
#pragma unroll
                    for (int t = 0; t < NT; ++t) Bn[t][k] = conv(t, u + 1, k, sc[t]);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int h = 0; h < MH; ++h) Ac[h] = An[h];
            }
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int k = 0; k < 4; ++k) Bc[t][k] = Bn[t][k];
        }
    };

    // ---- prologue: chunk cb's activations in buffer 0, its weights in W0,
    // chunk cb + 1's weights in flight into W1
    GmChunk<NT> W0, W1, W2;
    auto last = [&](int c) { return c < ce ? c : ce - 1; };
    xcopy(cb, 0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    wload(W0, cb);
    __builtin_amdgcn_sched_barrier(0);  // all of W0's loads ahead of W1's, as in the loop
    wload(W1, last(cb + 1));
    gm_vmwait<WLOADS>();
    __syncthreads();

    // step c (activation buffer b = (c - cb) % 2): the copies of chunk c + 1's
    // activations (buffer b ^ 1, read by no wave since the last barrier), the
    // weight loads of chunk c + 2 (two chunks ahead), then chunk c's math;
    // each wave waits for its own copies (the loads issued after them may
    // stay in flight) and the block barrier publishes them.  Past the range
    // the copies and loads repeat the last chunk (unconditional, in bounds),
    // so every wait count holds.  The compiler's own wait for Wc's loads
    // falls on gm_settle at the step's start (chunk c + 1's loads, issued
    // after Wc's, stay in flight).
    auto step = [&](int c, GmChunk<NT>& Wc, GmChunk<NT>& Wf) {
        const int b = (c - cb) & 1;
        gm_settle(Wc);
        xcopy(last(c + 1), b ^ 1);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        wload(Wf, last(c + 2));
        __builtin_amdgcn_sched_barrier(0);
        compute(Wc, b);
        gm_vmwait<WLOADS>();
        __syncthreads();
    };
    // whole rounds of three steps (no exits inside: the register sets keep
    // their places across the back edge), then the one or two left over
    const int nst = ce - cb;
    int c = cb;
    for (int i = 0; i < nst / 3; ++i, c += 3) {
        step(c, W0, W2);
        step(c + 1, W1, W0);
        step(c + 2, W2, W1);
    }
    if (nst % 3 >= 1) step(c, W0, W2);
    if (nst % 3 == 2) step(c + 1, W1, W0);
    gm_vmwait<0>();  // no copy may land in LDS after the block ends

    // ---- epilogue: acc[t][h][e] is activation row 32 h + 8 (e / 4) + 4 g + e % 4 of the group
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int h = 0; h < MH; ++h)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = 32 * h + 8 * (e >> 2) + 4 * g + (e & 3);
                if constexpr (SPLIT) {
                    if (valid[t] && m < Mz)
                        static_cast<float*>(Yv)[((int64_t)split * M + m0 + m) * nrows + row[t]] = acc[t][h][e];
                } else if constexpr (GU) {
                    const float up = __shfl_xor(acc[t][h][e], 16, 64);
                    if (valid[t] && n < 16 && m < Mz)
                        store_y<YT>(static_cast<YT*>(Yv) + (int64_t)(m0 + m) * nout + orow[t],
                                    silu_mul(acc[t][h][e], up));
                } else {
                    if (valid[t] && m < Mz)
                        store_y<YT>(static_cast<YT*>(Yv) + (int64_t)(m0 + m) * nout + orow[t], acc[t][h][e]);
                }
            }
}

template <int QT, int MH, int NT, int NW, bool GU>
hipError_t run_mid(const MidPlan& p, const WeightView& w, const bf16_t* x, void* y, bool yf32, int M, int64_t nout,
                   int64_t up_off, float* ws, hipStream_t s) {
    const int64_t per = GU ? 16 * NW * NT : 32 * NW * NT;  // outputs per block
    const int64_t tiles = (nout + per - 1) / per;
    const int64_t nb = tiles * p.splits * p.groups;
    if (nb > 0x7FFFFFFF) return hipErrorInvalidValue;
    const dim3 grid((unsigned)nb), block(64 * NW);
    const int K = (int)w.K, T = (int)tiles, S = p.splits;
    if (p.splits == 1) {
        if (yf32)
            hipLaunchKernelGGL((k_gemm_mid<QT, MH, NT, NW, GU, false, float>), grid, block, 0, s, w.q, x, y, M, K, nout,
                               up_off, w.N, p.cps, T, S);
        else
            hipLaunchKernelGGL((k_gemm_mid<QT, MH, NT, NW, GU, false, bf16_t>), grid, block, 0, s, w.q, x, y, M, K, nout,
                               up_off, w.N, p.cps, T, S);
        return hipGetLastError();
    }
    hipLaunchKernelGGL((k_gemm_mid<QT, MH, NT, NW, GU, true, float>), grid, block, 0, s, w.q, x, (void*)ws, M, K, nout,
                       up_off, w.N, p.cps, T, S);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_split_reduce(ws, y, yf32, GU, M, nout, up_off, w.N, p.splits, s);
}

template <int QT, int MH, int NT, int NW>
hipError_t run_mid_g(const MidPlan& p, const WeightView& w, const bf16_t* x, void* y, bool yf32, bool gu, int M,
                     int64_t nout, int64_t up_off, float* ws, hipStream_t s) {
    return gu ? run_mid<QT, MH, NT, NW, true>(p, w, x, y, yf32, M, nout, up_off, ws, s)
              : run_mid<QT, MH, NT, NW, false>(p, w, x, y, yf32, M, nout, up_off, ws, s);
}

}  // namespace

MidPlan plan_gemm_mid(int qtype, int64_t M, int64_t N, int64_t K, bool gu, int cus) {
    MidPlan p;
    if (!(qtype == 12 || qtype == 13)) return p;
    if (M < 1 || N < 1 || K < GM_KC || K % GM_KC || K > (int64_t)1 << 30 || (gu && N % 2)) return p;
    // 32-bit lane offsets: the row-quad plane and the activations below 4 GiB
    const uint64_t plane = (uint64_t)((N + 3) / 4) * (uint64_t)(K / 256) * 576u;
    if (plane >= (1ull << 32) || (uint64_t)M * (uint64_t)K * 2u >= (1ull << 32)) return p;
    const int64_t nch = K / GM_KC;
    // groups of 64 rows (MH = 2) or of 128 (MH = 4); NT 32-row column tiles
    // per wave, NW waves per block (blocks of 32 NW NT weight rows); two
    // resident 4-wave blocks per CU when MH NT <= 2, else one block.  Cost:
    // rounds of resident blocks x chunks per block x the measured time of a
    // round of one chunk (us, Q4_K 12288 x 4096 and 4096 x 12288 at
    // M = 128..512), plus per split 2 us and the f32 partials' round trip
    // at 4 TB/s.  THQ_MID_MH / THQ_MID_NT / THQ_MID_NW / THQ_MID_SPLITS
    // force the choice (tests, tuning).
    auto env_i = [](const char* n) {
        const char* e = getenv(n);
        return e && *e ? atoi(e) : 0;
    };
    const int fmh = env_i("THQ_MID_MH"), fnt = env_i("THQ_MID_NT"), fnw = env_i("THQ_MID_NW");
    const int forced = env_i("THQ_MID_SPLITS");
    const int64_t cu = cus > 0 ? cus : 256;
    const int64_t nout = gu ? N / 2 : N;
    struct Cfg {
        int mh, nt, nw, per_cu;
        double round_us;
    };
    static const Cfg cfgs[] = {{2, 1, 4, 2, 3.6}, {2, 2, 4, 1, 4.3}, {4, 1, 4, 1, 3.35},
                               {4, 2, 4, 1, 5.25}, {2, 1, 8, 1, 3.3}, {4, 1, 8, 1, 4.25}};
    double best = 1e30;
    int bs = 1, bmh = 2, bnt = 1, bnw = 4;
    for (const Cfg& f : cfgs) {
        if ((fmh && f.mh != fmh) || (fnt && f.nt != fnt) || (fnw && f.nw != fnw)) continue;
        const int64_t per = gu ? 16 * f.nw * f.nt : 32 * f.nw * f.nt;
        const int64_t tiles = (nout + per - 1) / per;
        const int64_t groups = (M + 32 * f.mh - 1) / (32 * f.mh);
        for (int s = 1; s <= 16 && s <= nch; ++s) {
            if (forced && s != (forced < nch ? forced : nch)) continue;
            const int64_t blocks = tiles * groups * s;
            const int64_t rounds = (blocks + cu * f.per_cu - 1) / (cu * f.per_cu);
            const int64_t cps = (nch + s - 1) / s;
            const double t = (double)rounds * (double)cps * f.round_us +
                             (s > 1 ? 2.0 + (double)s * (double)M * (double)N * 8.0 / 4.0e6 : 0.0);
            if (t < best - 1e-9) {
                best = t;
                bs = s;
                bmh = f.mh;
                bnt = f.nt;
                bnw = f.nw;
            }
        }
    }
    p.mh = bmh;
    p.nt = bnt;
    p.nw = bnw;
    p.groups = (int)((M + 32 * p.mh - 1) / (32 * p.mh));
    p.cps = (int)((nch + bs - 1) / bs);
    p.splits = (int)((nch + p.cps - 1) / p.cps);
    p.workspace_bytes = p.splits > 1 ? (size_t)p.splits * (size_t)M * (size_t)N * 4u : 0;
    return p;
}

hipError_t launch_gemm_mid(const MidPlan& p, const WeightView& w, const void* x, void* y, bool yf32, bool gu, int M,
                           int64_t nout, int64_t up_off, float* ws, hipStream_t s) {
    if (p.splits < 1 || p.groups < 1 || M < 1 || (p.splits > 1 && !ws)) return hipErrorInvalidValue;
    const bf16_t* xb = static_cast<const bf16_t*>(x);
    if (w.qtype != 12 && w.qtype != 13) return hipErrorInvalidValue;
    auto go = [&](auto mh, auto nt, auto nw) {
        constexpr int MH = decltype(mh)::value, NT = decltype(nt)::value, NW = decltype(nw)::value;
        return w.qtype == 13 ? run_mid_g<13, MH, NT, NW>(p, w, xb, y, yf32, gu, M, nout, up_off, ws, s)
                             : run_mid_g<12, MH, NT, NW>(p, w, xb, y, yf32, gu, M, nout, up_off, ws, s);
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I4 = std::integral_constant<int, 4>;
    using I8 = std::integral_constant<int, 8>;
    if (p.nw == 8) {
        if (p.mh == 2 && p.nt == 1) return go(I2{}, I1{}, I8{});
        if (p.mh == 4 && p.nt == 1) return go(I4{}, I1{}, I8{});
        return hipErrorInvalidValue;
    }
    if (p.nw != 4) return hipErrorInvalidValue;
    if (p.mh == 2 && p.nt == 1) return go(I2{}, I1{}, I4{});
    if (p.mh == 2 && p.nt == 2) return go(I2{}, I2{}, I4{});
    if (p.mh == 4 && p.nt == 1) return go(I4{}, I1{}, I4{});
    if (p.mh == 4 && p.nt == 2) return go(I4{}, I2{}, I4{});
    return hipErrorInvalidValue;
}

}  // namespace thq
