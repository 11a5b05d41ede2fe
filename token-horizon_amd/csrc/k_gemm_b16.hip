// k_gemm_b16.hip — bf16 x bf16 GEMM for the dequantize-then-GEMM prefill
// route: y[M, N] = x[M, K] . Wb[N, K]^T, f32 accumulation, where Wb is the
// weight dequantized to bf16 once per call (launch_dequant_*).
//
// Role: the reference router's "dequant + bf16 matmul" prefill route
// (pf_route, engine/src/quant_kernel.rs:5117-5300, with AffineDequant
// :1035-1040 writing the bf16 scratch).  For large M this beats
// dequantizing inside the GEMM tile (k_gemm_fq.hip): a 512-row tile repeats
// the conversion once per row block (4 times at M = 2048), about 62 VALU
// instructions per wave per 32-wide K step that the MFMAs do not fully
// hide, while one pass over the weights costs about 25 us.
//
// Tiling: block tile 256 (M) x 384 (N) x 64 (K), 8 waves (two per SIMD) as
// 2 (M) x 4 (N), wave tile 128 x 96 of v_mfma_f32_32x32x16_bf16 (192 f32
// accumulators per lane).  Each wave reads one set of fragments per 16-wide
// k group and runs its 12 MFMAs, 48 per K step; the SIMD's other wave
// covers the LDS latency.  Operands come in by direct-to-LDS copies
// (global_load_lds_dwordx4) into 2 slots (160 KB), the next K step's copies
// issued right after the barrier that frees their slot, with 128-B LDS rows
// whose 16-B chunks are XOR-swizzled (chunk c of row r at slot
// c ^ ((r >> 1) & 7): any 16 consecutive rows at one chunk hit 16 distinct
// bank groups).  One block barrier per 64-wide K step (a 32-wide step with a
// 3-slot ring, one barrier per 32: 2048 x 12288 x 4096 in 211 against 174 us,
// 4096 x 12288 x 4096 356 against 322 us, weights streamed from HBM).
// Blocks are dealt to the 8 XCDs round-robin; the grid is renumbered so each XCD runs a contiguous range of tiles, 8 row
// blocks x all column blocks at a time: at M = 2048 an XCD's 32 tiles are
// all 8 row blocks of 4 column blocks, so each bf16 weight byte leaves HBM
// once (x, 6x smaller, once per XCD; 4 row blocks x 8 column blocks fetched
// W twice: 268 against 235 MB, 2 % slower).  Rows past M or N copy a clamped row
// and are never stored.  Offsets are 32-bit: the router keeps x and Wb
// below 4 GiB.
#include "thq_dev.hpp"
#include "thq_kernels.hpp"

namespace thq {
namespace {

constexpr int GB_BM = 256, GB_BN = 384, GB_BK = 64, GB_NS = 2;

__device__ __forceinline__ uint32_t gb_lds(const void* p) {
    return (uint32_t)(size_t)(__attribute__((address_space(3))) const void*)p;
}
// 16 bytes per lane from base + voff to LDS at m0 + 16 * lane.  Inline asm:
// the compiler's wait insertion would otherwise put a vmcnt(0) before every
// LDS read that follows a direct-to-LDS load, serializing the ring.
__device__ __forceinline__ void gb_dma16(uint32_t lds, const void* base, uint32_t voff) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"{m0}"(lds), "v"(voff), "s"(base) : "memory");
}
template <int N>
__device__ __forceinline__ void gb_wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ int gb_slot(int r, int c) { return c ^ ((r >> 1) & 7); }
__device__ __forceinline__ int gb_swz(int r, int c) { return r * GB_BK + (gb_slot(r, c) << 3); }
__device__ __forceinline__ f32x16_t gb_mfma(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// linear block -> (row block, column block): XCD x = b & 7 runs a contiguous
// range of linear tiles, ordered in groups of 8 row blocks x all column
// blocks (row blocks fastest within a group)
__device__ __forceinline__ void gb_tile(int tiles_n, int tiles_m, int& tn, int& tm) {
    const int nb = gridDim.x, b = blockIdx.x;
    const int q = (nb + 7) >> 3, tall = (nb & 7) ? (nb & 7) : 8;
    const int xcd = b & 7, local = b >> 3;
    const int L = xcd < tall ? xcd * q + local : tall * q + (xcd - tall) * (q - 1) + local;
    constexpr int GM = 8;
    const int grp = L / (GM * tiles_n), r = L % (GM * tiles_n);
    const int rows_in = tiles_m - grp * GM < GM ? tiles_m - grp * GM : GM;  // the last group may be short
    tm = grp * GM + r % rows_in;
    tn = r / rows_in;
}

template <typename YT>
__global__ __launch_bounds__(512) void k_gemm_b16(const bf16_t* __restrict__ X, const bf16_t* __restrict__ W,
                                                 YT* __restrict__ Y, int M, int N, int K, int tiles_n,
                                                 int tiles_m) {
    constexpr int TM = 128, TN = 96, MT = 4, NT = 3;
    constexpr int WNV = GB_BN / TN;         // 4 waves along N
    constexpr int XI = GB_BM * 8 / 512;     // X copies per wave per step (16-B chunks / 64 lanes / 8 waves)
    constexpr int WI = GB_BN * 8 / 512;     // W copies per wave per step
    __shared__ __attribute__((aligned(16))) bf16_t Xs[GB_NS][GB_BM * GB_BK];
    __shared__ __attribute__((aligned(16))) bf16_t Ws[GB_NS][GB_BN * GB_BK];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WNV, wn = wave % WNV;
    int tn, tm;
    gb_tile(tiles_n, tiles_m, tn, tm);
    const int m0 = tm * GB_BM, n0 = tn * GB_BN;
    const int T = K / GB_BK;
    // copy descriptors: instruction i of this wave covers 8 rows; lane ->
    // row lane / 8, LDS slot lane % 8, which holds chunk gb_slot(row, slot)
    uint32_t xoff[XI], woff[WI];
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const int r = wave * (GB_BM / 8) + 8 * i + (lane >> 3);
        int m = m0 + r;
        if (m >= M) m = M - 1;
        xoff[i] = (uint32_t)(((int64_t)m * K + 8 * gb_slot(r, lane & 7)) * 2);
    }
#pragma unroll
    for (int i = 0; i < WI; ++i) {
        const int r = wave * (GB_BN / 8) + 8 * i + (lane >> 3);
        int n = n0 + r;
        if (n >= N) n = N - 1;
        woff[i] = (uint32_t)(((int64_t)n * K + 8 * gb_slot(r, lane & 7)) * 2);
    }
    const uint32_t xl = gb_lds(&Xs[0][0]) + wave * (GB_BM / 8) * GB_BK * 2;
    const uint32_t wl = gb_lds(&Ws[0][0]) + wave * (GB_BN / 8) * GB_BK * 2;
    auto copy = [&](int t) {
        const int s = t % GB_NS;
#pragma unroll
        for (int i = 0; i < XI; ++i) gb_dma16(xl + s * (GB_BM * GB_BK * 2) + i * 1024, X + t * GB_BK, xoff[i]);
#pragma unroll
        for (int i = 0; i < WI; ++i) gb_dma16(wl + s * (GB_BN * GB_BK * 2) + i * 1024, W + t * GB_BK, woff[i]);
    };
    const int lr = lane & 31, lh = lane >> 5;
    f32x16_t acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    if (T > 0) copy(0);
    for (int t = 0; t < T; ++t) {
        // step t's copies have landed, for every wave (they are the only ones
        // in flight); after the barrier every wave is past step t - 1, so
        // slot (t + 1) % 2 is free for step t + 1
        gb_wait_vm<0>();
        __syncthreads();
        if (t + 1 < T) copy(t + 1);
        const bf16_t* xs = &Xs[t % GB_NS][0];
        const bf16_t* ws = &Ws[t % GB_NS][0];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const int ch = 2 * kk + lh;
            bf16x8_t a[MT], b[NT];
#pragma unroll
            for (int i = 0; i < MT; ++i)
                a[i] = *reinterpret_cast<const bf16x8_t*>(xs + gb_swz(wm * TM + 32 * i + lr, ch));
#pragma unroll
            for (int j = 0; j < NT; ++j)
                b[j] = *reinterpret_cast<const bf16x8_t*>(ws + gb_swz(wn * TN + 32 * j + lr, ch));
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < NT; ++j) acc[i][j] = gb_mfma(a[i], b[j], acc[i][j]);
        }
    }
    // lane holds column lr of each 32 x 32 tile, rows 8 (e / 4) + 4 (lane / 32) + e % 4
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int m = m0 + wm * TM + 32 * i + 8 * (e >> 2) + 4 * lh + (e & 3);
            if (m >= M) continue;
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const int n = n0 + wn * TN + 32 * j + lr;
                if (n < N) store_y<YT>(Y + (int64_t)m * N + n, acc[i][j][e]);
            }
        }
}

}  // namespace

int64_t gemm_b16_blocks(int64_t M, int64_t N) { return ((M + GB_BM - 1) / GB_BM) * ((N + GB_BN - 1) / GB_BN); }

bool gemm_b16_supported(int64_t M, int64_t N, int64_t K) {
    return M >= 1 && N >= 1 && K >= GB_BK && K % GB_BK == 0 && (uint64_t)M * (uint64_t)K * 2 < (1ull << 32) &&
           (uint64_t)N * (uint64_t)K * 2 < (1ull << 32) && M < (1 << 30) && N < (1 << 30);
}

hipError_t launch_gemm_b16(const void* x, const void* wb, void* y, bool yf32, int M, int N, int K, hipStream_t s) {
    const int tiles_m = (M + GB_BM - 1) / GB_BM, tiles_n = (N + GB_BN - 1) / GB_BN;
    const dim3 grid((unsigned)(tiles_m * tiles_n));
    const bf16_t* xb = static_cast<const bf16_t*>(x);
    const bf16_t* wbb = static_cast<const bf16_t*>(wb);
    if (yf32)
        hipLaunchKernelGGL(k_gemm_b16<float>, grid, dim3(512), 0, s, xb, wbb, static_cast<float*>(y), M, N, K, tiles_n,
                           tiles_m);
    else
        hipLaunchKernelGGL(k_gemm_b16<bf16_t>, grid, dim3(512), 0, s, xb, wbb, static_cast<bf16_t*>(y), M, N, K,
                           tiles_n, tiles_m);
    return hipGetLastError();
}

}  // namespace thq
