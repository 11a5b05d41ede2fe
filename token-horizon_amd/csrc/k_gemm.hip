// k_gemm.hip — prefill / speculative-verify GEMM for gfx950:
// y[M, N] = x[M, K] (bf16) . W[N, K]^T with W in GGUF Q4_K or Q8_0 blocks.
//
// Role: the m > 8 projections of the reference (AffineQpf / AffineQmppPrefill,
// engine/src/quant_kernel.rs:3740-5095, routed by pf_route :5117) over GGUF
// weights; fused gate/up with the silu(gate)*up epilogue
// (engine/src/quant_kernel.rs:2922-2926).
//
// Tiling: block tile BM x 128 (N) x 64 (K), 4 waves as 2 (M) x 2 (N), wave
// tile (BM/2) x 64 made of 32x32 v_mfma_f32_32x32x16_bf16 tiles.  Each K step
// the block dequantizes a 128 x 64 W tile into LDS as bf16 (one 16-32 B
// vector of packed weights per thread) while the MFMAs consume the previous
// tile: two LDS buffers, one barrier per K step.
//
// Two weight modes:
//   rounded  W tile = bf16(d*sc*q - dmin*m)         (Q4_K, Q8_0; large M)
//   exact    W tile = bf16(q) (exact for |q| <= 255) and the f32 block scale
//            is applied to each 32-wide partial in registers (Q8_0), so the
//            result carries no weight rounding (LM head / argmax).  Q4_K and
//            MLX affine: W tile = bf16(128 + q) (exact), and each 32-wide
//            sub-block's partial A enters the total as d1*A - c1*S with
//            c1 = 128*d1 + m1 (Q4_K: d1 = d*sc, m1 = dmin*m; affine:
//            d1 = scale, m1 = -bias) and S the sub-block's sum of each x row,
//            taken while x is stored to LDS.
// Split-K: grid.z splits write f32 partials that k_split_reduce sums in a
// fixed order (deterministic), applying the same epilogue.
#include "thq_dev.hpp"
#include "thq_kernels.hpp"

namespace thq {

constexpr int BN = 128;
constexpr int BK = 64;
constexpr int LDK = BK + 8;  // padded LDS row (bf16 elements): 144 B

__device__ __forceinline__ f32x16_t mfma32(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// W-tile column c (0..127) -> weight row; in gate/up mode each wave's 64
// columns are 32 gate rows followed by the 32 up rows of the same outputs.
template <bool GU>
__device__ __forceinline__ int64_t tile_row(int c, int64_t bx, int64_t nout, int64_t up_off, bool& valid) {
    if (GU) {
        const int wn = c >> 6, tn = (c >> 5) & 1, j = c & 31;
        const int64_t i = bx * 64 + 32 * wn + j;
        valid = i < nout;
        return i + (tn ? up_off : 0);
    }
    const int64_t r = bx * BN + c;
    valid = r < nout;
    return r;
}

// 8 packed nibbles (one per byte, bits 0..3) -> d1*q - m1 as 4 bf16 pairs
__device__ __forceinline__ void deq8_q4(uint32_t w, float d1, float m1, uint32_t* out) {
    const float f0 = ubyte_f32<0>(w), f1 = ubyte_f32<1>(w);
    const float f2 = ubyte_f32<2>(w), f3 = ubyte_f32<3>(w);
    out[0] = pack_bf16x2(__builtin_fmaf(d1, f0, -m1), __builtin_fmaf(d1, f1, -m1));
    out[1] = pack_bf16x2(__builtin_fmaf(d1, f2, -m1), __builtin_fmaf(d1, f3, -m1));
}

template <int QT, bool EXACT, int BM, bool GU, typename YT, bool SPLIT>
__global__ __launch_bounds__(256) void k_gemm(const uint8_t* __restrict__ Wq, const uint8_t* __restrict__ Wa,
                                             const bf16_t* __restrict__ X, void* __restrict__ Yv, int M, int K,
                                             int64_t nout, int64_t up_off, int64_t ldy, int kiters_per_split) {
    constexpr int TM = BM / 2;   // wave tile rows (M)
    constexpr int MT = TM / 32;  // 32-row MFMA tiles per wave
    constexpr int XCH = BM * 8 / 256;  // 16-B X chunks per thread per K step
    __shared__ __attribute__((aligned(16))) bf16_t Xs[2][BM][LDK];
    __shared__ __attribute__((aligned(16))) bf16_t Ws[2][BN][LDK];
    __shared__ float Ds[2][BN][2];
    // exact Q4_K / affine: per W-tile row {d1, c1} of the step's two 32-wide
    // sub-blocks, and per x row the two sub-block sums (row-contiguous)
    constexpr bool XQ4 = EXACT && QT != 8;
    __shared__ float Dq[XQ4 ? 2 : 1][XQ4 ? BN : 1][4];
    __shared__ __attribute__((aligned(16))) float Sx[XQ4 ? 2 : 1][2][XQ4 ? BM : 4];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t bx = blockIdx.x;
    const int64_t m0 = (int64_t)blockIdx.y * BM;
    const int kit0 = blockIdx.z * kiters_per_split;
    int kit1 = kit0 + kiters_per_split;
    const int kiters = K / BK;
    if (kit1 > kiters) kit1 = kiters;

    // this thread's W-tile row and half
    const int wc = tid >> 1, wh = tid & 1;
    bool wvalid;
    const int64_t wrow = tile_row<GU>(wc, bx, nout, up_off, wvalid);

    uint4 xr[XCH];
    uint4 wr0, wr1;     // packed weights
    uint4 hdr;          // Q4_K superblock header
    uint16_t dq = 0;    // Q8_0 block scale

    auto gload = [&](int kit) {
        const int k0 = kit * BK;
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            const int c = tid + 256 * i;
            const int row = c >> 3, col8 = c & 7;
            const int64_t m = m0 + row;
            if (m < M)
                xr[i] = *reinterpret_cast<const uint4*>(X + m * K + k0 + 8 * col8);
            else
                xr[i] = make_uint4(0, 0, 0, 0);
        }
        if (!wvalid) {
            wr0 = wr1 = hdr = make_uint4(0, 0, 0, 0);
            dq = 0;
            return;
        }
        if (QT != 8) {
            const int nsb = K >> 8, sidx = k0 >> 8, j = (k0 & 255) >> 6;
            hdr.x = *reinterpret_cast<const uint32_t*>(Wq + q4k_hdword(wrow, nsb, sidx, 0));
            hdr.y = *reinterpret_cast<const uint32_t*>(Wq + q4k_hdword(wrow, nsb, sidx, 1));
            hdr.z = *reinterpret_cast<const uint32_t*>(Wq + q4k_hdword(wrow, nsb, sidx, 2));
            hdr.w = *reinterpret_cast<const uint32_t*>(Wq + q4k_hdword(wrow, nsb, sidx, 3));
            wr0 = *reinterpret_cast<const uint4*>(Wq + q4k_piece(wrow, nsb, sidx, wh, j));
        } else {
            const int64_t blk = (k0 >> 5) + wh;
            wr0 = *reinterpret_cast<const uint4*>(Wq + q8t_q(wrow, K >> 5, blk, 0));
            wr1 = *reinterpret_cast<const uint4*>(Wq + q8t_q(wrow, K >> 5, blk, 1));
            dq = reinterpret_cast<const uint16_t*>(Wa)[q8t_d(wrow, K >> 5, blk)];
        }
    };

    auto lstore = [&](int buf, int kit) {
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            const int c = tid + 256 * i;
            *reinterpret_cast<uint4*>(&Xs[buf][c >> 3][8 * (c & 7)]) = xr[i];
            if constexpr (XQ4) {
                // 32-wide sums: four consecutive threads hold one sub-block
                const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
                bf16x2_t q2[4];
                __builtin_memcpy(q2, &xr[i], 16);
                float t = __builtin_amdgcn_fdot2_f32_bf16(q2[0], one, 0.0f, false);
                t = __builtin_amdgcn_fdot2_f32_bf16(q2[1], one, t, false);
                t = __builtin_amdgcn_fdot2_f32_bf16(q2[2], one, t, false);
                t = __builtin_amdgcn_fdot2_f32_bf16(q2[3], one, t, false);
                t += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(t), 0xB1, 0xF, 0xF, false));
                t += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(t), 0x4E, 0xF, 0xF, false));
                if ((c & 3) == 0) Sx[buf][(c >> 2) & 1][c >> 3] = t;
            }
        }
        if (QT != 8) {
            const int j = ((kit * BK) & 255) >> 6;
            float d1, m1, d2, m2;
            if constexpr (QT == 13) {  // affine group: w = scale * q + bias
                const uint32_t hw = j == 0 ? hdr.x : (j == 1 ? hdr.y : (j == 2 ? hdr.z : hdr.w));
                d1 = d2 = aff_scale(hw);
                m1 = m2 = -aff_bias(hw);
            } else {
                uint32_t sc0, mm0, sc1, mm1;
                q4k_hdr_sm(hdr, 2 * j, sc0, mm0);
                q4k_hdr_sm(hdr, 2 * j + 1, sc1, mm1);
                const float d = q4k_hdr_d(hdr), dmin = q4k_hdr_dmin(hdr);
                d1 = d * (float)sc0;
                m1 = dmin * (float)mm0;
                d2 = d * (float)sc1;
                m2 = dmin * (float)mm1;
            }
            const uint32_t q[4] = {wr0.x, wr0.y, wr0.z, wr0.w};
            uint32_t lo[8], hi[8];
            if constexpr (XQ4) {
                // bf16(128 + q): the nibble in the low mantissa bits under a 0x43 byte
                const uint32_t C43 = 0x43434343u;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint32_t l4 = q[t] & 0x0F0F0F0Fu, h4 = (q[t] >> 4) & 0x0F0F0F0Fu;
                    lo[2 * t] = __builtin_amdgcn_perm(C43, l4, 0x04010400u);
                    lo[2 * t + 1] = __builtin_amdgcn_perm(C43, l4, 0x04030402u);
                    hi[2 * t] = __builtin_amdgcn_perm(C43, h4, 0x04010400u);
                    hi[2 * t + 1] = __builtin_amdgcn_perm(C43, h4, 0x04030402u);
                }
                if (wh == 0)
                    *reinterpret_cast<float4*>(&Dq[buf][wc][0]) = make_float4(
                        d1, __builtin_fmaf(128.0f, d1, m1), d2, __builtin_fmaf(128.0f, d2, m2));
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    deq8_q4(q[t] & 0x0F0F0F0Fu, d1, m1, lo + 2 * t);
                    deq8_q4((q[t] >> 4) & 0x0F0F0F0Fu, d2, m2, hi + 2 * t);
                }
            }
            uint4* dl = reinterpret_cast<uint4*>(&Ws[buf][wc][16 * wh]);
            uint4* dh = reinterpret_cast<uint4*>(&Ws[buf][wc][32 + 16 * wh]);
            dl[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            dl[1] = make_uint4(lo[4], lo[5], lo[6], lo[7]);
            dh[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            dh[1] = make_uint4(hi[4], hi[5], hi[6], hi[7]);
        } else {
            const uint32_t q[8] = {wr0.x, wr0.y, wr0.z, wr0.w, wr1.x, wr1.y, wr1.z, wr1.w};
            const float d = f16_to_f32(dq);
            uint32_t o[16];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const float f0 = (float)(int8_t)(q[t] & 0xFF), f1 = (float)(int8_t)((q[t] >> 8) & 0xFF);
                const float f2 = (float)(int8_t)((q[t] >> 16) & 0xFF), f3 = (float)(int8_t)(q[t] >> 24);
                if (EXACT) {
                    o[2 * t] = pack_bf16x2(f0, f1);
                    o[2 * t + 1] = pack_bf16x2(f2, f3);
                } else {
                    o[2 * t] = pack_bf16x2(f0 * d, f1 * d);
                    o[2 * t + 1] = pack_bf16x2(f2 * d, f3 * d);
                }
            }
            uint4* dst = reinterpret_cast<uint4*>(&Ws[buf][wc][32 * wh]);
#pragma unroll
            for (int v = 0; v < 4; ++v) dst[v] = make_uint4(o[4 * v], o[4 * v + 1], o[4 * v + 2], o[4 * v + 3]);
            if (EXACT) Ds[buf][wc][wh] = d;
        }
    };

    f32x16_t acc[MT][2];
    f32x16_t tot[MT][2];
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                acc[a][b][i] = 0.0f;
                tot[a][b][i] = 0.0f;
            }

    if (kit0 < kit1) {
        gload(kit0);
        lstore(0, kit0);
    }
    __syncthreads();
    const int lr = lane & 31, lk = 8 * (lane >> 5);
    for (int kit = kit0; kit < kit1; ++kit) {
        const int buf = (kit - kit0) & 1;
        const bool more = kit + 1 < kit1;
        if (more) gload(kit + 1);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            bf16x8_t a[MT], b[2];
#pragma unroll
            for (int t = 0; t < MT; ++t)
                a[t] = *reinterpret_cast<const bf16x8_t*>(&Xs[buf][wm * TM + 32 * t + lr][16 * kk + lk]);
#pragma unroll
            for (int t = 0; t < 2; ++t)
                b[t] = *reinterpret_cast<const bf16x8_t*>(&Ws[buf][wn * 64 + 32 * t + lr][16 * kk + lk]);
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma32(a[i], b[j], acc[i][j]);
            if (XQ4 && (kk & 1)) {
                // end of a 32-wide sub-block: tot += d1 * A - c1 * S
                const int sb = kk >> 1;
                f32x4_t sv[MT][4];
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int g4 = 0; g4 < 4; ++g4)
                        sv[i][g4] = *reinterpret_cast<const f32x4_t*>(&Sx[buf][sb][wm * TM + 32 * i + 8 * g4 + 4 * (lane >> 5)]);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float2 dc = *reinterpret_cast<const float2*>(&Dq[buf][wn * 64 + 32 * j + lr][2 * sb]);
#pragma unroll
                    for (int i = 0; i < MT; ++i)
#pragma unroll
                        for (int e = 0; e < 16; ++e) {
                            const float t = __builtin_fmaf(dc.x, acc[i][j][e], tot[i][j][e]);
                            tot[i][j][e] = __builtin_fmaf(-dc.y, sv[i][e >> 2][e & 3], t);
                            acc[i][j][e] = 0.0f;
                        }
                }
            } else if (EXACT && (kk & 1)) {
                // end of a 32-wide block: scale the partial into the total
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float ds = Ds[buf][wn * 64 + 32 * j + lr][kk >> 1];
#pragma unroll
                    for (int i = 0; i < MT; ++i)
#pragma unroll
                        for (int e = 0; e < 16; ++e) {
                            tot[i][j][e] = __builtin_fmaf(ds, acc[i][j][e], tot[i][j][e]);
                            acc[i][j][e] = 0.0f;
                        }
                }
            }
        }
        if (more) lstore(buf ^ 1, kit + 1);
        __syncthreads();
    }
    if (!EXACT) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) tot[i][j] = acc[i][j];
    }

    // epilogue: lane holds column lr of each 32x32 tile, rows 8*(e/4) + 4*(lane/32) + e%4
    const int rq = 4 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int64_t m = m0 + wm * TM + 32 * i + 8 * (e >> 2) + rq + (e & 3);
            if (m >= M) continue;
            if (GU) {
                const int64_t o = bx * 64 + 32 * wn + lr;
                if (o >= nout) continue;
                if (SPLIT) {
                    float* P = static_cast<float*>(Yv) + (int64_t)blockIdx.z * M * ldy;
                    P[m * ldy + o] = tot[i][0][e];
                    P[m * ldy + up_off + o] = tot[i][1][e];
                } else {
                    store_y<YT>(static_cast<YT*>(Yv) + m * ldy + o, silu_mul(tot[i][0][e], tot[i][1][e]));
                }
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int64_t n = bx * BN + wn * 64 + 32 * j + lr;
                    if (n >= nout) continue;
                    if (SPLIT)
                        (static_cast<float*>(Yv) + (int64_t)blockIdx.z * M * ldy)[m * ldy + n] = tot[i][j][e];
                    else
                        store_y<YT>(static_cast<YT*>(Yv) + m * ldy + n, tot[i][j][e]);
                }
            }
        }
    }
}

// ------------------------------------------------------------------ streamed GEMM (rounded weights)
// The production kernel for bf16 activations with rounded weight tiles.
// Every global read is a direct-to-LDS copy (global_load_lds_dword[x4]),
// issued two K steps ahead of its use, so no register holds in-flight data
// and each wave waits on its own copies with one explicit s_waitcnt per
// K step, followed by the block barrier:
//   X ring      3 slots of BM x 64 bf16, rows of 128 B with 16-B chunk c of
//               row r at chunk slot c ^ (r & 7) (conflict-free MFMA operand
//               reads); rows past M copy row M-1 and are never stored
//   raw W ring  3 slots of the packed 128 x 64 weight tile as stored in HBM
//               (Q4_K: 32 B of nibbles + the 16-B header per row; Q8_0: 64 B
//               of int8 + one dword of two f16 scales per row)
//   W tiles     2 bf16 buffers, swizzled like X; while the MFMAs of step t
//               read one, step t+1's raw tile is dequantized into the other,
//               a quarter after each 16-wide MFMA round
// The copies are written as inline asm because the compiler's own wait
// insertion treats any LDS access after a direct-to-LDS load as dependent on
// it (a vmcnt(0) before every LDS read), which would serialize the ring.
// Block order: blocks are dealt round-robin to the 8 XCDs; the grid is
// renumbered so that each XCD runs a contiguous range of tiles (tiles along N
// fastest), keeping its X rows in its own L2.
// Offsets are 32-bit: the host routes X or weight planes of 4 GiB and more to
// k_gemm.

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(size_t)(__attribute__((address_space(3))) const void*)p;
}
// 16 (x4) or 4 bytes per lane from base + voff to LDS at m0 + 16*lane (4*lane)
__device__ __forceinline__ void dma16(uint32_t lds, const void* base, uint32_t voff) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"{m0}"(lds), "v"(voff), "s"(base) : "memory");
}
__device__ __forceinline__ void dma4(uint32_t lds, const void* base, uint32_t voff) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %1, %2" ::"{m0}"(lds), "v"(voff), "s"(base) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// LDS has 64 banks of 4 B: 16 lanes of a b128 access share a cycle, i.e. two
// 128-B rows per bank row.  Chunk c of row r sits at slot c ^ ((r >> 1) & 7),
// so any 16 consecutive rows at one chunk hit 16 distinct 16-B bank groups.
__device__ __forceinline__ int swz_slot(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }
__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + (swz_slot(row, chunk) << 3); }

// linear block -> (x, y, z) tile, contiguous ranges per XCD
__device__ __forceinline__ void xcd_tile(int tiles_n, int tiles_m, int& x, int& y, int& z) {
    const int nb = gridDim.x, b = blockIdx.x;
    const int q = (nb + 7) >> 3, tall = (nb & 7) ? (nb & 7) : 8;
    const int xcd = b & 7, local = b >> 3;
    const int L = xcd < tall ? xcd * q + local : tall * q + (xcd - tall) * (q - 1) + local;
    x = L % tiles_n;
    y = (L / tiles_n) % tiles_m;
    z = L / (tiles_n * tiles_m);
}

template <int QT, int BM, int WM, bool GU, typename YT, bool SPLIT>
__global__ __launch_bounds__(128 * WM) void k_gemm_dma(const uint8_t* __restrict__ Wq, const uint8_t* __restrict__ Wa,
                                                      const bf16_t* __restrict__ X, void* __restrict__ Yv, int M, int K,
                                                      int64_t nout, int64_t up_off, int64_t ldy, int kiters_per_split,
                                                      int tiles_n, int tiles_m) {
    // waves: WM (along M) x 2 (along N); wave tile TM x 64
    constexpr int NW = 2 * WM;
    constexpr int TM = BM / WM;
    constexpr int MT = TM / 32;
    static_assert(MT >= 1 && (NW == 4 || NW == 8), "tile configuration");
    // copies per wave per K step: X = 8*BM 16-B slots over NW waves; packed
    // weights: Q4_K 256 slots of nibbles + 512 header dwords, Q8_0 512 slots
    // of int8 + 128 scale dwords, Q6_K 384 slots (QL low / high piece, QH
    // piece of each row) + 128 scale dwords + 128 dwords holding d, spread so
    // that every wave issues the same number of copies (some with part of
    // the wave active)
    constexpr bool Q6 = QT == 14;
    constexpr int XI = BM / (8 * NW);
    constexpr int NIB = Q6 ? BN * 48 : (QT != 8 ? BN * 32 : BN * 64);  // packed weight bytes per raw slot
    constexpr int AUX = Q6 ? BN * 8 : (QT != 8 ? BN * 16 : BN * 4);    // header / scale bytes per raw slot
    constexpr int RAW = NIB + AUX;
    constexpr int NSLOT = (Q6 ? 384 : (QT != 8 ? 256 : 512)) / NW;   // 16-B weight slots per wave
    constexpr int NI = (NSLOT + 63) / 64;                            // their copies
    constexpr int NL = NSLOT / NI;                                   // active lanes per copy
    constexpr int HSLOT = (Q6 ? 256 : (QT != 8 ? 512 : 128)) / NW;   // header / scale dwords per wave
    constexpr int HI = (HSLOT + 63) / 64;
    constexpr int HL = HSLOT / HI;
    constexpr int WI = NI + HI;
    static_assert(XI >= 1 && NI * NL == NSLOT && HI * HL == HSLOT, "copy split");
    __shared__ __attribute__((aligned(16))) bf16_t Xs[3][BM * BK];
    __shared__ __attribute__((aligned(16))) bf16_t Ws[2][BN * BK];
    __shared__ __attribute__((aligned(16))) uint8_t Wr[3][RAW];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    int bxi, byi, bzi;
    xcd_tile(tiles_n, tiles_m, bxi, byi, bzi);
    const int64_t bx = bxi;
    const int64_t m0 = (int64_t)byi * BM;
    const int kit0 = bzi * kiters_per_split;
    const int kiters = K / BK;
    const int kit1 = kit0 + kiters_per_split < kiters ? kit0 + kiters_per_split : kiters;
    const int T = kit1 > kit0 ? kit1 - kit0 : 0;
    const int nsb = K >> 8;

    // ---- copy descriptors (per-lane 32-bit offsets, per-wave LDS bases)
    uint32_t xoff[XI];
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        // lane -> row r, LDS slot lane & 7, which holds chunk swz_slot(r, lane & 7)
        const int r = wave * (BM / NW) + 8 * i + (lane >> 3);
        const int c = swz_slot(r, lane & 7);
        int64_t m = m0 + r;
        if (m >= M) m = M - 1;
        xoff[i] = (uint32_t)((m * K + 8 * c) * 2);
    }
    const uint32_t xlds = lds_addr(&Xs[0][0]) + wave * (BM / NW) * 128;
    const uint32_t wlds = lds_addr(&Wr[0][0]);
    auto clamp_row = [&](int c) {
        bool v;
        const int64_t r = tile_row<GU>(c, bx, nout, up_off, v);
        return v ? r : (int64_t)0;
    };
    // packed weights: Q4_K slot j = h*128 + row (piece h of the row),
    // Q8_0 slot j = (half*2 + c)*128 + row (bytes 32*half + 16*c .. +15),
    // Q6_K slot j = p*128 + row (p = 0, 1: QL bytes 16p .. 16p+15 of the
    // step, p = 2: its 16 QH bytes); headers: Q4_K dword j = row*4 + p, Q8_0
    // dword j = row (two f16 scales), Q6_K dword j = row (the step's 4
    // scales) and 128 + row (the dword holding the superblock's f16 d)
    const Q6Layout q6l = q6k_layout(Q6 ? (GU ? 2 * up_off : nout) : 0, K);
    uint32_t noff[NI], hoff[HI], nstr[NI], hq[HI];
    bool hd[HI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int j = wave * NSLOT + NL * i + (lane < NL ? lane : 0);
        const int row = j & 127, hc = j >> 7;
        if (Q6) {
            noff[i] = hc < 2 ? (uint32_t)(clamp_row(row) * (K >> 1) + 16 * hc)
                             : (uint32_t)(q6l.qh + clamp_row(row) * (K >> 2));
            nstr[i] = hc < 2 ? 32u : 16u;  // bytes per K step
        } else if (QT != 8) {
            noff[i] = (uint32_t)q4k_piece(clamp_row(row), nsb, 0, hc, 0);
        } else {
            // Q8_0 tiles: block 2 kit + (hc >> 1), half hc & 1; the step adds 2048 kit
            noff[i] = (uint32_t)q8t_q(clamp_row(row), K >> 5, hc >> 1, hc & 1);
        }
    }
#pragma unroll
    for (int i = 0; i < HI; ++i) {
        const int j = wave * HSLOT + HL * i + (lane < HL ? lane : 0);
        hd[i] = false;
        if (Q6) {
            hd[i] = j >= 128;
            const int64_t r = clamp_row(j & 127);
            hoff[i] = (uint32_t)(q6l.sc + r * (K >> 4));
            hq[i] = (uint32_t)(r * nsb);
        } else if (QT != 8) {
            hoff[i] = (uint32_t)q4k_hdword(clamp_row(j >> 2), nsb, 0, j & 3);
        } else {
            // the dword of blocks 2 kit, 2 kit + 1 in the row's scale chunk kit / 4
            hoff[i] = (uint32_t)(q8t_d(clamp_row(j), K >> 5, 0) * 2);
        }
    }
    auto xcopy = [&](int kit, int slot) {
        const bf16_t* base = X + kit * BK;
#pragma unroll
        for (int i = 0; i < XI; ++i) dma16(xlds + slot * (BM * BK * 2) + i * 1024, base, xoff[i]);
    };
    auto wcopy = [&](int kit, int slot) {
        const uint32_t l = wlds + slot * RAW;
        const uint8_t* nb = Q6 ? Wq : (QT != 8 ? Wq + kit * 16 : Wq + kit * 2048);
        const uint8_t* hb = Q6 ? Wq : (QT != 8 ? Wq + (kit >> 2) * 64 : Wa + (kit >> 2) * 512 + (kit & 3) * 4);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const uint32_t off = Q6 ? noff[i] + (uint32_t)kit * nstr[i] : noff[i];
            if (NL == 64 || lane < NL) dma16(l + (wave * NSLOT + NL * i) * 16, nb, off);
        }
#pragma unroll
        for (int i = 0; i < HI; ++i) {
            // Q6_K d: the dword holding f16 number r*nsb + kit/4 of the D plane
            const uint32_t off = !Q6 ? hoff[i]
                                     : (hd[i] ? (uint32_t)q6l.d + (((hq[i] + (uint32_t)(kit >> 2)) * 2u) & ~3u)
                                              : hoff[i] + 4u * (uint32_t)kit);
            if (HL == 64 || lane < HL) dma4(l + NIB + (wave * HSLOT + HL * i) * 4, hb, off);
        }
    };

    // ---- dequantization: thread -> tile row wc and (wave-uniform) part q:
    // 4 waves: q = piece / half wh, quarters 0..3; 8 waves: piece / half
    // wh = q >> 1, quarters 2*(q & 1) + {0, 1}
    constexpr int QPT = 16 / NW;  // quarters (8 weights) per thread per K step
    const int wc = tid & (BN - 1), q = tid >> 7;
    const int wh = NW == 4 ? q : q >> 1;
    const int qbase = NW == 4 ? 0 : 2 * (q & 1);
    bool wvalid;
    const int64_t wrow = tile_row<GU>(wc, bx, nout, up_off, wvalid);
    const uint32_t wpar = Q6 ? (uint32_t)((wvalid ? wrow : 0) * nsb) & 1u : 0u;  // parity of the row's first d
    // Per K step each thread converts 32 weights.  Byte -> f32 goes through
    // v_perm_b32 with an exponent byte (no int->float conversion):
    //   Q4_K nibble q:   bytes [0, 0, q, 0x43]        = 128 + q
    //                    w = fma(d1, 128 + q, -(128*d1 + m1))
    //   Q8_0 int8 q:     u = q ^ 0x80 (0..255); bytes [0, u, 0, 0x47]
    //                    = 2^15 + u;  w = fma(d, that, -(2^15 + 128)*d) = d*q
    // (the high byte keeps the exponent's low bit clear, so the value byte
    // sits in mantissa bits only; (2^15 + 128)*d = 257*128*d is exact in f32,
    // so the Q8_0 result is exact; Q4_K differs from d1*q - m1 by far less
    // than the bf16 rounding that follows).
    //   Q6_K code c:     bytes [0, 0, c, 0x43]        = 128 + c
    //                    w = fma(s, 128 + c, -160*s) = s*(c - 32), s = d*sc,
    //                    exact before the bf16 rounding (one rounding, as
    //                    the product (d*sc)*(c - 32))
    struct Raw {
        uint4 q0, q1;
        uint4 h;               // Q6_K QH bytes of the step
        float s0, c0, s1, c1;  // scale and offset of the tile row's two 32-weight halves (Q6_K: 16-weight groups)
    };
    auto rload = [&](int slot, int kit) {
        Raw R;
        const uint8_t* w = &Wr[slot][0];
        if constexpr (Q6) {
            // 4 waves: thread half wh covers step weights 32wh .. +31 (QL pieces 0, 1,
            // groups 2wh, 2wh + 1); 8 waves: weights 32wh + 16(q & 1) .. +15 (QL piece q & 1,
            // group 2wh + (q & 1))
            R.q0 = *reinterpret_cast<const uint4*>(w + ((NW == 4 ? 0 : (q & 1)) * BN + wc) * 16);
            R.q1 = NW == 4 ? *reinterpret_cast<const uint4*>(w + (BN + wc) * 16) : R.q0;
            R.h = *reinterpret_cast<const uint4*>(w + (2 * BN + wc) * 16);
            const uint32_t scw = *reinterpret_cast<const uint32_t*>(w + NIB + wc * 4);
            const uint32_t dw = *reinterpret_cast<const uint32_t*>(w + NIB + (BN + wc) * 4);
            float d = f16_to_f32((uint16_t)(((wpar ^ ((uint32_t)kit >> 2)) & 1u) ? dw >> 16 : dw));
            if (!wvalid) d = 0.0f;
            const int g0 = NW == 4 ? 2 * wh : 2 * wh + (q & 1);
            R.s0 = d * (float)(int)(int8_t)(scw >> (8 * g0));
            R.s1 = NW == 4 ? d * (float)(int)(int8_t)(scw >> (8 * g0 + 8)) : R.s0;
            R.c0 = 160.0f * R.s0;
            R.c1 = 160.0f * R.s1;
        } else if (QT != 8) {
            R.q0 = *reinterpret_cast<const uint4*>(w + (wh * BN + wc) * 16);
            R.q1 = R.q0;
            const uint32_t hw = *reinterpret_cast<const uint32_t*>(w + NIB + wc * 16 + (kit & 3) * 4);
            if constexpr (QT == 13) {  // affine group: w = scale * (128 + q) - (128 * scale - bias)
                const float sc = wvalid ? aff_scale(hw) : 0.0f, bi = wvalid ? aff_bias(hw) : 0.0f;
                R.s0 = R.s1 = sc;
                R.c0 = R.c1 = __builtin_fmaf(128.0f, sc, -bi);
            } else {
                const uint4 h = *reinterpret_cast<const uint4*>(w + NIB + wc * 16);
                float d = q4k_hdr_d(h), dm = q4k_hdr_dmin(h);
                if (!wvalid) d = dm = 0.0f;
                R.s0 = d * (float)(hw & 63u);
                R.c0 = __builtin_fmaf(128.0f, R.s0, dm * (float)((hw >> 6) & 63u));
                R.s1 = d * (float)((hw >> 12) & 63u);
                R.c1 = __builtin_fmaf(128.0f, R.s1, dm * (float)((hw >> 18) & 63u));
            }
        } else {
            // 4 waves: both 16-B pieces of the half; 8 waves: only piece q & 1
            R.q0 = *reinterpret_cast<const uint4*>(w + ((wh * 2 + (NW == 4 ? 0 : (q & 1))) * BN + wc) * 16);
            R.q1 = NW == 4 ? *reinterpret_cast<const uint4*>(w + ((wh * 2 + 1) * BN + wc) * 16) : R.q0;
            const uint32_t sc = *reinterpret_cast<const uint32_t*>(w + NIB + wc * 4);
            float d = f16_to_f32((uint16_t)(wh ? sc >> 16 : sc));
            if (!wvalid) d = 0.0f;
            R.s0 = R.s1 = d;
            R.c0 = R.c1 = 32896.0f * d;
        }
        return R;
    };
    // the thread's quarter k (0 .. QPT-1, compile-time): 8 weights -> one 16-B chunk
    auto dequant = [&](const Raw& R, int buf, int k) {
        bf16_t* wt = &Ws[buf][0];
        uint32_t a, b;
        float sc, c;
        int ch;
        uint32_t E;
        if constexpr (Q6) {
            // chunk k: weights w0 .. w0+7 of the step, 4 waves w0 = 32wh + 8k,
            // 8 waves w0 = 32wh + 16(q & 1) + 8k; codes from QL bytes w0 % 32 ..
            // (nibble wh) and QH bytes w0 % 16 .. (field w0 / 16)
            const uint4 src = (NW == 4 && k >= 2) ? R.q1 : R.q0;
            const int sel = k & 1;
            const uint32_t qa = sel ? src.z : src.x, qb = sel ? src.w : src.y;
            const uint32_t ha = sel ? R.h.z : R.h.x, hb = sel ? R.h.w : R.h.y;
            const int grp = NW == 4 ? 2 * wh + (k >> 1) : 2 * wh + (q & 1);
            const int ns = 4 * wh, hs = 2 * grp;
            a = ((qa >> ns) & 0x0F0F0F0Fu) | (((ha >> hs) & 0x03030303u) << 4);
            b = ((qb >> ns) & 0x0F0F0F0Fu) | (((hb >> hs) & 0x03030303u) << 4);
            sc = (NW == 4 && k >= 2) ? R.s1 : R.s0;
            c = (NW == 4 && k >= 2) ? R.c1 : R.c0;
            ch = NW == 4 ? 4 * wh + k : 4 * wh + 2 * (q & 1) + k;
            E = 0x43434343u;
        } else if (QT != 8) {
            // low nibbles = first 32 weights of the step, high = second 32; 4 waves:
            // quarters 0,1 low and 2,3 high; 8 waves: the half is q & 1
            const int hi = NW == 4 ? (k >> 1) : (q & 1);
            const int sel = NW == 4 ? (k & 1) : k;
            const uint32_t qa = sel ? R.q0.z : R.q0.x, qb = sel ? R.q0.w : R.q0.y;
            a = (qa >> (4 * hi)) & 0x0F0F0F0Fu;
            b = (qb >> (4 * hi)) & 0x0F0F0F0Fu;
            sc = hi ? R.s1 : R.s0;
            c = hi ? R.c1 : R.c0;
            ch = 4 * hi + 2 * wh + sel;
            E = 0x43434343u;
        } else {
            // 4 waves: quarters 0,1 from q0 and 2,3 from q1; 8 waves: both from q0
            const uint4 src = (NW == 4 && k >= 2) ? R.q1 : R.q0;
            const int sel = NW == 4 ? (k & 1) : k;
            a = (sel ? src.z : src.x) ^ 0x80808080u;
            b = (sel ? src.w : src.y) ^ 0x80808080u;
            sc = R.s0;
            c = R.c0;
            ch = 4 * wh + qbase + k;
            E = 0x47474747u;
        }
        // byte i of v into byte 2 (Q4_K) or byte 1 (Q8_0), exponent byte from E
        auto f = [&](uint32_t v, int i) {
            const uint32_t sel = QT != 8 ? 0x04000c0cu | ((uint32_t)i << 16) : 0x040c000cu | ((uint32_t)i << 8);
            return __builtin_fmaf(sc, __uint_as_float(__builtin_amdgcn_perm(E, v, sel)), -c);
        };
        const uint32_t o0 = pack_bf16x2(f(a, 0), f(a, 1));
        const uint32_t o1 = pack_bf16x2(f(a, 2), f(a, 3));
        const uint32_t o2 = pack_bf16x2(f(b, 0), f(b, 1));
        const uint32_t o3 = pack_bf16x2(f(b, 2), f(b, 3));
        *reinterpret_cast<uint4*>(wt + swz(wc, ch)) = make_uint4(o0, o1, o2, o3);
    };

    f32x16_t acc[MT][2];
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;

    const int lr = lane & 31, lhalf = lane >> 5;
    // MFMAs of one K step on X slot xs / W buffer wb; with has_next, the raw
    // tile in slot rs (step kn) is dequantized into W buffer wb ^ 1
    auto step = [&](int xs, int wb, bool has_next, int rs, int kn) {
        const bf16_t* xt = &Xs[xs][0];
        const bf16_t* wt = &Ws[wb][0];
        // every operand fragment of the step is requested up front so the LDS
        // latency overlaps the first MFMAs
        bf16x8_t a[4][MT], b[4][2];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const int ch = 2 * kk + lhalf;
#pragma unroll
            for (int t = 0; t < MT; ++t)
                a[kk][t] = *reinterpret_cast<const bf16x8_t*>(xt + swz(wm * TM + 32 * t + lr, ch));
#pragma unroll
            for (int t = 0; t < 2; ++t) b[kk][t] = *reinterpret_cast<const bf16x8_t*>(wt + swz(wn * 64 + 32 * t + lr, ch));
        }
        Raw R;
        if (has_next) R = rload(rs, kn);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma32(a[kk][i], b[kk][j], acc[i][j]);
            if (has_next && (kk % (4 / QPT)) == (4 / QPT) - 1) dequant(R, wb ^ 1, kk / (4 / QPT));
        }
    };

    if (T > 0) {
        // prologue: X(0), raw(0), raw(1), X(1), raw(2).  Step 0 reads X(0)
        // and dequantizes raw(1), so everything up to raw(1) must land here;
        // X(1) and raw(2) stay in flight
        xcopy(kit0, 0);
        wcopy(kit0, 0);
        if (T > 1) {
            wcopy(kit0 + 1, 1);
            xcopy(kit0 + 1, 1);
        }
        if (T > 2) wcopy(kit0 + 2, 2);
        if (T > 2) wait_vm<XI + WI>();
        else if (T > 1) wait_vm<XI>();
        else wait_vm<0>();
        __syncthreads();
        {
            const Raw R = rload(0, kit0);
#pragma unroll
            for (int k = 0; k < QPT; ++k) dequant(R, 0, k);
        }
        __syncthreads();
    }
    int xs = 0, rs = 1;  // X slot of step t, raw slot of step t + 1
    int t = 0;
    // steady state: X two steps ahead into slot (t + 2) % 3, raw W three
    // steps ahead into slot (t + 3) % 3 == t % 3
    for (; t + 3 < T; ++t) {
        xcopy(kit0 + t + 2, xs == 0 ? 2 : xs - 1);
        wcopy(kit0 + t + 3, xs);
        step(xs, t & 1, true, rs, kit0 + t + 1);
        wait_vm<XI + WI>();
        __syncthreads();
        xs = xs == 2 ? 0 : xs + 1;
        rs = rs == 2 ? 0 : rs + 1;
    }
    // last (up to) three steps
    for (; t < T; ++t) {
        const bool px = t + 2 < T;
        if (px) xcopy(kit0 + t + 2, xs == 0 ? 2 : xs - 1);
        step(xs, t & 1, t + 1 < T, rs, kit0 + t + 1);
        if (px) wait_vm<XI>();
        else wait_vm<0>();
        __syncthreads();
        xs = xs == 2 ? 0 : xs + 1;
        rs = rs == 2 ? 0 : rs + 1;
    }

    // epilogue: lane holds column lr of each 32x32 tile, rows 8*(e/4) + 4*(lane/32) + e%4
    const int rq = 4 * lhalf;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int64_t m = m0 + wm * TM + 32 * i + 8 * (e >> 2) + rq + (e & 3);
            if (m >= M) continue;
            if (GU) {
                const int64_t o = bx * 64 + 32 * wn + lr;
                if (o >= nout) continue;
                if (SPLIT) {
                    float* P = static_cast<float*>(Yv) + (int64_t)bzi * M * ldy;
                    P[m * ldy + o] = acc[i][0][e];
                    P[m * ldy + up_off + o] = acc[i][1][e];
                } else {
                    store_y<YT>(static_cast<YT*>(Yv) + m * ldy + o, silu_mul(acc[i][0][e], acc[i][1][e]));
                }
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int64_t n = bx * BN + wn * 64 + 32 * j + lr;
                    if (n >= nout) continue;
                    if (SPLIT)
                        (static_cast<float*>(Yv) + (int64_t)bzi * M * ldy)[m * ldy + n] = acc[i][j][e];
                    else
                        store_y<YT>(static_cast<YT*>(Yv) + m * ldy + n, acc[i][j][e]);
                }
            }
        }
    }
}

// sum split partials P[s][M][ldp] in split order, then the epilogue
template <bool GU, typename YT>
__global__ __launch_bounds__(256) void k_split_reduce(const float* __restrict__ P, YT* __restrict__ y, int M,
                                                     int64_t nout, int64_t up_off, int64_t ldp, int splits) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)M * nout) return;
    const int64_t m = t / nout, o = t - m * nout;
    float g = 0.0f, u = 0.0f;
    for (int s = 0; s < splits; ++s) {
        const float* Ps = P + (int64_t)s * M * ldp + m * ldp;
        g += Ps[o];
        if (GU) u += Ps[up_off + o];
    }
    store_y<YT>(y + m * nout + o, GU ? silu_mul(g, u) : g);
}

// The same sums, four outputs per thread with 16-B loads (nout, ldp and
// up_off multiples of 4, P and y 16-B aligned), the loads of four splits
// issued before their adds: each element is still summed in split order
// from 0, so the bits equal k_split_reduce's.
template <bool GU, typename YT>
__global__ __launch_bounds__(256) void k_split_reduce4(const float* __restrict__ P, YT* __restrict__ y, int M,
                                                      int64_t nout, int64_t up_off, int64_t ldp, int splits) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t q = nout >> 2;
    if (t >= (int64_t)M * q) return;
    const int64_t m = t / q, o = (t - m * q) * 4;
    const float* base = P + m * ldp + o;
    const int64_t ss = (int64_t)M * ldp;  // split stride
    f32x4_t g = {0.0f, 0.0f, 0.0f, 0.0f}, u = {0.0f, 0.0f, 0.0f, 0.0f};
    int sp = 0;
    for (; sp + 4 <= splits; sp += 4) {
        f32x4_t a[4], b[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            a[j] = *reinterpret_cast<const f32x4_t*>(base + (int64_t)(sp + j) * ss);
            if (GU) b[j] = *reinterpret_cast<const f32x4_t*>(base + (int64_t)(sp + j) * ss + up_off);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            g += a[j];
            if (GU) u += b[j];
        }
    }
    for (; sp < splits; ++sp) {
        g += *reinterpret_cast<const f32x4_t*>(base + (int64_t)sp * ss);
        if (GU) u += *reinterpret_cast<const f32x4_t*>(base + (int64_t)sp * ss + up_off);
    }
    YT* yo = y + m * nout + o;
#pragma unroll
    for (int i = 0; i < 4; ++i) store_y<YT>(yo + i, GU ? silu_mul(g[i], u[i]) : g[i]);
}

hipError_t launch_split_reduce(const float* P, void* y, bool yf32, bool gu, int M, int64_t nout, int64_t up_off,
                               int64_t ldp, int splits, hipStream_t s) {
    const int64_t total = (int64_t)M * nout;
    const bool vec = nout % 4 == 0 && ldp % 4 == 0 && up_off % 4 == 0 && (uintptr_t)P % 16 == 0 &&
                     (uintptr_t)y % 16 == 0;
    if (vec) {
        const dim3 grid4((unsigned)((total / 4 + 255) / 256));
        if (gu) {
            if (yf32) hipLaunchKernelGGL((k_split_reduce4<true, float>), grid4, dim3(256), 0, s, P, (float*)y, M, nout, up_off, ldp, splits);
            else hipLaunchKernelGGL((k_split_reduce4<true, bf16_t>), grid4, dim3(256), 0, s, P, (bf16_t*)y, M, nout, up_off, ldp, splits);
        } else {
            if (yf32) hipLaunchKernelGGL((k_split_reduce4<false, float>), grid4, dim3(256), 0, s, P, (float*)y, M, nout, up_off, ldp, splits);
            else hipLaunchKernelGGL((k_split_reduce4<false, bf16_t>), grid4, dim3(256), 0, s, P, (bf16_t*)y, M, nout, up_off, ldp, splits);
        }
        return hipGetLastError();
    }
    const dim3 grid((unsigned)((total + 255) / 256));
    if (gu) {
        if (yf32) hipLaunchKernelGGL((k_split_reduce<true, float>), grid, dim3(256), 0, s, P, (float*)y, M, nout, up_off, ldp, splits);
        else hipLaunchKernelGGL((k_split_reduce<true, bf16_t>), grid, dim3(256), 0, s, P, (bf16_t*)y, M, nout, up_off, ldp, splits);
    } else {
        if (yf32) hipLaunchKernelGGL((k_split_reduce<false, float>), grid, dim3(256), 0, s, P, (float*)y, M, nout, up_off, ldp, splits);
        else hipLaunchKernelGGL((k_split_reduce<false, bf16_t>), grid, dim3(256), 0, s, P, (bf16_t*)y, M, nout, up_off, ldp, splits);
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ launch
static inline int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

// K-split count for the 128- and 256-row tiles.  Their blocks hold more than
// 80 KB of LDS, so one block per CU is resident.  The modeled time is:
//   rounds of resident blocks x K steps per block x step time
//   + per split, the partials' round trip through HBM (written once, read
//     once by k_split_reduce: 8 B per output element) and the reduce launch.
// Step times were measured on MI355X with every CU busy: 1.25 us for 256-row
// tiles, 1.1 us for 128-row tiles.  The partials are priced at 5 TB/s.  On
// the 9 swept Q4_K shapes (M = 128..1024; 12288 x 4096 and 4096 x 12288;
// counts 1, 2, 3, 4, 8 timed), the model picks the fastest count every time.
static int pick_splits(int64_t blocks, int kiters, int max_split, int64_t M, int64_t N_rows, int bm, int cus) {
    const double tstep = bm == 256 ? 1.25 : 1.1;                    // us per K step
    const double part = (double)M * (double)N_rows * 8.0 / 5.0e6;  // us per split
    int best = 1;
    double best_t = 0.0;
    for (int s = 1; s <= max_split && s <= 64; ++s) {
        const int kps = (kiters + s - 1) / s;
        if ((kiters + kps - 1) / kps != s) continue;  // the same plan as a smaller count
        const int64_t rounds = (blocks * s + cus - 1) / cus;
        const double t = (double)rounds * kps * tstep + (s > 1 ? s * part + 2.0 : 0.0);
        if (s == 1 || t < best_t) {
            best = s;
            best_t = t;
        }
    }
    return best;
}

GemmPlan plan_gemm(int qtype, bool exact, int64_t M, int64_t N_rows, int64_t K, bool gu, int cus) {
    GemmPlan p;
    if (cus < 1) cus = 256;
    int bm = env_int("THQ_GEMM_BM", 0);
    if (bm != 64 && bm != 128 && bm != 256) bm = M <= 64 ? 64 : (M <= 128 ? 128 : 256);
    if (exact && bm > 64) bm = 64;  // the exact tile keeps two accumulator sets
    p.bm = bm;
    const int64_t nout = gu ? N_rows / 2 : N_rows;
    p.tiles_n = gu ? (nout + 63) / 64 : (nout + BN - 1) / BN;
    p.tiles_m = (M + bm - 1) / bm;
    const int kiters = (int)(K / BK);
    if (kiters < 1) {
        // K < 64: no GEMM tiles (the router sends such K to the generic
        // kernel); an empty plan keeps workspace sizing well defined
        p.kps = 0;
        p.splits = 1;
        p.workspace_bytes = 0;
        return p;
    }
    int splits = env_int("THQ_GEMM_SPLITS", 0);
    if (splits <= 0) {
        const int64_t blocks = p.tiles_n * p.tiles_m;
        const int max_split = kiters / 2 > 0 ? kiters / 2 : 1;
        splits = 1;
        if (bm == 64) {
            // 64-row tiles (< 80 KB of LDS): two blocks per CU.  Split K as far
            // as the grid still fits one round of resident blocks: a partial
            // second round costs a whole round of K steps (12288 x 4096 at
            // M = 16..64: 5 splits 25.0-29.6 us, 6 splits 29.8-35.3 us)
            const int64_t slots = 2 * (int64_t)cus;
            if (blocks < slots) {
                splits = (int)(slots / blocks);
                if (splits > max_split) splits = max_split;
            }
        } else {
            splits = pick_splits(blocks, kiters, max_split, M, N_rows, bm, cus);
        }
    }
    if (splits > kiters) splits = kiters;
    if (splits < 1) splits = 1;
    p.kps = (kiters + splits - 1) / splits;
    p.splits = (kiters + p.kps - 1) / p.kps;
    p.workspace_bytes = p.splits > 1 ? (size_t)p.splits * (size_t)M * (size_t)N_rows * sizeof(float) : 0;
    return p;
}

template <int QT, bool EXACT, int BM, bool GU, typename YT>
static hipError_t gemm_t(const GemmPlan& p, const WeightView& w, const bf16_t* x, void* y, int M, float* ws,
                         hipStream_t s) {
    const int64_t nout = GU ? w.N / 2 : w.N;
    const int64_t up_off = GU ? w.N / 2 : 0;
    dim3 grid((unsigned)p.tiles_n, (unsigned)p.tiles_m, (unsigned)p.splits);
    const uint64_t xbytes = (uint64_t)M * (uint64_t)w.K * 2;
    const uint64_t wbytes = QT == 14  ? (uint64_t)q6k_layout(w.N, w.K).total
                            : QT != 8 ? (uint64_t)((w.N + 3) / 4) * (uint64_t)(w.K / 256) * 576
                                      : (uint64_t)w.N * (uint64_t)w.K;
    if constexpr (QT == 14) {
        // Q6_K runs the DMA kernel only (32-bit copy offsets, rounded weights)
        if (EXACT || xbytes >= (1ull << 32) || wbytes >= (1ull << 32)) return hipErrorInvalidValue;
    }
    if (QT == 14 || (!EXACT && xbytes < (1ull << 32) && wbytes < (1ull << 32) && !env_int("THQ_GEMM_V1", 0))) {
        const unsigned nb = (unsigned)(p.tiles_n * p.tiles_m * p.splits);
        constexpr int WM = BM == 64 ? 2 : 4;  // 8 waves (2 per SIMD) for the large tiles
        if (p.splits == 1) {
            hipLaunchKernelGGL((k_gemm_dma<QT, BM, WM, GU, YT, false>), dim3(nb), dim3(128 * WM), 0, s, w.q, w.aux,
                               x, y, M, (int)w.K, nout, up_off, nout, p.kps, (int)p.tiles_n, (int)p.tiles_m);
            return hipGetLastError();
        }
        hipLaunchKernelGGL((k_gemm_dma<QT, BM, WM, GU, float, true>), dim3(nb), dim3(128 * WM), 0, s, w.q, w.aux, x,
                           (void*)ws, M, (int)w.K, nout, up_off, (int64_t)w.N, p.kps, (int)p.tiles_n,
                           (int)p.tiles_m);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_split_reduce(ws, y, std::is_same<YT, float>::value, GU, M, nout, up_off, (int64_t)w.N,
                                   p.splits, s);
    }
    if constexpr (QT == 14) {
        return hipErrorInvalidValue;
    } else {
        if (p.splits == 1) {
            hipLaunchKernelGGL((k_gemm<QT, EXACT, BM, GU, YT, false>), grid, dim3(256), 0, s, w.q, w.aux, x, y, M,
                               (int)w.K, nout, up_off, nout, p.kps);
            return hipGetLastError();
        }
        // partials in natural weight-row order: ld = N rows
        hipLaunchKernelGGL((k_gemm<QT, EXACT, BM, GU, float, true>), grid, dim3(256), 0, s, w.q, w.aux, x, (void*)ws,
                           M, (int)w.K, nout, up_off, (int64_t)w.N, p.kps);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_split_reduce(ws, y, std::is_same<YT, float>::value, GU, M, nout, up_off, (int64_t)w.N,
                                   p.splits, s);
    }
}

template <int QT, bool EXACT, bool GU, typename YT>
static hipError_t gemm_bm(const GemmPlan& p, const WeightView& w, const bf16_t* x, void* y, int M, float* ws,
                          hipStream_t s) {
    if constexpr (EXACT) {
        return gemm_t<QT, EXACT, 64, GU, YT>(p, w, x, y, M, ws, s);
    } else {
        if (p.bm == 64) return gemm_t<QT, EXACT, 64, GU, YT>(p, w, x, y, M, ws, s);
        if (p.bm == 128) return gemm_t<QT, EXACT, 128, GU, YT>(p, w, x, y, M, ws, s);
        return gemm_t<QT, EXACT, 256, GU, YT>(p, w, x, y, M, ws, s);
    }
}

hipError_t launch_gemm(const GemmPlan& p, const WeightView& w, const void* x, void* y, bool yf32, bool gu, bool exact,
                       int M, float* ws, hipStream_t s) {
    const bf16_t* xb = static_cast<const bf16_t*>(x);
    if (w.qtype == 12) {
        if (exact) {
            if (gu) return yf32 ? gemm_bm<12, true, true, float>(p, w, xb, y, M, ws, s)
                                : gemm_bm<12, true, true, bf16_t>(p, w, xb, y, M, ws, s);
            return yf32 ? gemm_bm<12, true, false, float>(p, w, xb, y, M, ws, s)
                        : gemm_bm<12, true, false, bf16_t>(p, w, xb, y, M, ws, s);
        }
        if (gu) return yf32 ? gemm_bm<12, false, true, float>(p, w, xb, y, M, ws, s)
                            : gemm_bm<12, false, true, bf16_t>(p, w, xb, y, M, ws, s);
        return yf32 ? gemm_bm<12, false, false, float>(p, w, xb, y, M, ws, s)
                    : gemm_bm<12, false, false, bf16_t>(p, w, xb, y, M, ws, s);
    }
    if (w.qtype == 13) {
        if (exact) {
            if (gu) return yf32 ? gemm_bm<13, true, true, float>(p, w, xb, y, M, ws, s)
                                : gemm_bm<13, true, true, bf16_t>(p, w, xb, y, M, ws, s);
            return yf32 ? gemm_bm<13, true, false, float>(p, w, xb, y, M, ws, s)
                        : gemm_bm<13, true, false, bf16_t>(p, w, xb, y, M, ws, s);
        }
        if (gu) return yf32 ? gemm_bm<13, false, true, float>(p, w, xb, y, M, ws, s)
                            : gemm_bm<13, false, true, bf16_t>(p, w, xb, y, M, ws, s);
        return yf32 ? gemm_bm<13, false, false, float>(p, w, xb, y, M, ws, s)
                    : gemm_bm<13, false, false, bf16_t>(p, w, xb, y, M, ws, s);
    }
    if (w.qtype == 14) {
        if (exact) return hipErrorInvalidValue;
        if (gu) return yf32 ? gemm_bm<14, false, true, float>(p, w, xb, y, M, ws, s)
                            : gemm_bm<14, false, true, bf16_t>(p, w, xb, y, M, ws, s);
        return yf32 ? gemm_bm<14, false, false, float>(p, w, xb, y, M, ws, s)
                    : gemm_bm<14, false, false, bf16_t>(p, w, xb, y, M, ws, s);
    }
    if (exact) {
        if (gu) return yf32 ? gemm_bm<8, true, true, float>(p, w, xb, y, M, ws, s)
                            : gemm_bm<8, true, true, bf16_t>(p, w, xb, y, M, ws, s);
        return yf32 ? gemm_bm<8, true, false, float>(p, w, xb, y, M, ws, s)
                    : gemm_bm<8, true, false, bf16_t>(p, w, xb, y, M, ws, s);
    }
    if (gu) return yf32 ? gemm_bm<8, false, true, float>(p, w, xb, y, M, ws, s)
                        : gemm_bm<8, false, true, bf16_t>(p, w, xb, y, M, ws, s);
    return yf32 ? gemm_bm<8, false, false, float>(p, w, xb, y, M, ws, s)
                : gemm_bm<8, false, false, bf16_t>(p, w, xb, y, M, ws, s);
}

}  // namespace thq
