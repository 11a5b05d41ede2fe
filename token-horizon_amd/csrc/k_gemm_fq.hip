// k_gemm_fq.hip — prefill / verify GEMM with the 4-bit weight dequantized
// into LDS inside the tile: y[M, N] = x[M, K] (bf16) . W[N, K]^T, W in the
// Q4_K or MLX-affine row-quad layout, f32 accumulation on
// v_mfma_f32_32x32x16_bf16.
//
// Role: the reference's large-M prefill route (pf_route -> pf_policy_large ->
// AffineQpf, engine/src/quant_kernel.rs:5117-5145, 5206-5211: the weight
// tile dequantized to bf16 in threadgroup memory and contracted on the
// matrix units), over GGUF Q4_K and the engine's MLX affine 4-bit weights;
// the fused gate/up with the silu(gate)*up epilogue
// (engine/src/quant_kernel.rs:2922-2926).
//
// Weight values: each weight is bf16(d1*q - m1) rounded to nearest even,
// with d1*q - m1 formed in f32 by one fma (d1 = d*sc and m1 = dmin*m are
// exact products of an f16 and a 6-bit integer; d1*q is exact too), i.e.
// exactly the bf16 of the bit-exact f32 dequantization.  MLX affine:
// bf16(fma(scale, q, bias)).
//
// K order.  A K step is 32 weights of a row: the 16-B nibble piece
// (h, s, p) of the row-quad layout, i.e. positions 16h .. 16h+15 of
// sub-blocks 2p (low nibbles) and 2p+1 (high nibbles) of superblock s.
// Step t = 8s + 4h + p, so the four steps of a "quad" Q = 2s + h read the
// row's four consecutive pieces (h, s, 0..3): 64 contiguous bytes, copied
// once per quad.  Inside the step, k-slot j < 16 is column
// 256s + 64p + 16h + j and k-slot 16 + j is column 256s + 64p + 32 + 16h + j;
// the x tile is copied in that order (16-B chunks of columns +0, +8, +32,
// +40), so the contraction is over the same pairs as x . W^T, summed in
// another order.
//
// Tiling: block tile BM x BN x 32 with BM = 32 WM MT, BN = 32 WN NT; 8 waves
// (two per SIMD) as WM x WN of (32 MT) x (32 NT) wave tiles.  Per step:
//   x      direct-to-LDS copies (global_load_lds_dwordx4) into a 3-slot ring,
//          two steps ahead; 64-B rows with XOR-swizzled 16-B chunks
//   raw W  direct-to-LDS copies into an RS-slot ring, RS - 1 quads (4 steps
//          each) ahead: per row its 64 B of nibble pieces, per row quad its
//          64 B of header dwords [p][r] for superblock s
//   (waves 0..3 issue the x copies and waves 4..7 the raw ones, each wave
//   waiting only on its own stream)
//   W      2 bf16 tiles swizzled like x: while the MFMAs of step t read one,
//          the block converts the raw tile of step t + 1 into the other, two
//          lanes per weight row (each decodes the row's scales and writes 16
//          weights as two 16-B chunks), the conversion interleaved with the
//          step's MFMAs
// One block barrier per step.  Blocks are dealt round-robin to the 8 XCDs;
// the grid is renumbered so each XCD runs a contiguous range of tiles in
// groups of 8 row blocks x all column blocks (K splits slowest).  Rows past M
// copy row M-1 and rows past N a clamped row; neither is stored.  Offsets are
// 32-bit: the router keeps x and the weight plane below 4 GiB.
// Split K (SPLIT): split z covers steps [z kps, (z + 1) kps) and writes f32
// partials [z][M][ldy] that k_split_reduce sums in split order.
#include <type_traits>

#include "thq_dev.hpp"
#include "thq_kernels.hpp"

namespace thq {
namespace {

constexpr int FQ_BK = 32;
constexpr int FQ_VPM = 6;  // VALU instructions issued after each MFMA of a step

__device__ __forceinline__ uint32_t fq_lds(const void* p) {
    return (uint32_t)(size_t)(__attribute__((address_space(3))) const void*)p;
}
// 16 bytes per active lane from base + voff to LDS at m0 + 16 * lane.  Inline
// asm: the compiler's wait insertion would otherwise put a vmcnt(0) before
// every LDS read that follows a direct-to-LDS load, serializing the rings.
__device__ __forceinline__ void fq_dma16(uint32_t lds, const void* base, uint32_t voff) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"{m0}"(lds), "v"(voff), "s"(base) : "memory");
}
template <int N>
__device__ __forceinline__ void fq_wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// chunk c of row r at chunk slot c ^ ((r >> 2) & 3): 16 consecutive rows at
// one chunk hit 16 distinct 16-B bank groups
__device__ __forceinline__ int fq_slot(int r, int c) { return c ^ ((r >> 2) & 3); }
__device__ __forceinline__ int fq_swz(int r, int c) { return r * FQ_BK + (fq_slot(r, c) << 3); }
__device__ __forceinline__ f32x16_t fq_mfma(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// linear block -> (row block, column block, split): XCD x = b & 7 runs a
// contiguous range of linear tiles; within a split, groups of 8 row blocks x
// all column blocks, row blocks fastest
__device__ __forceinline__ void fq_tile(int tiles_n, int tiles_m, int& tn, int& tm, int& tz) {
    const int nb = gridDim.x, b = blockIdx.x;
    const int q = (nb + 7) >> 3, tall = (nb & 7) ? (nb & 7) : 8;
    const int xcd = b & 7, local = b >> 3;
    int L = xcd < tall ? xcd * q + local : tall * q + (xcd - tall) * (q - 1) + local;
    const int per = tiles_n * tiles_m;
    tz = L / per;
    L -= tz * per;
    constexpr int GM = 8;
    const int grp = L / (GM * tiles_n), r = L % (GM * tiles_n);
    const int rows_in = tiles_m - grp * GM < GM ? tiles_m - grp * GM : GM;
    tm = grp * GM + r % rows_in;
    tn = r / rows_in;
}

// tile column c -> weight row (valid = an output of this call); gate/up: each
// wave's 64 columns are 32 gate rows then the 32 up rows of the same outputs
template <bool GU, int TN>
__device__ __forceinline__ int64_t fq_row(int c, int tn, int bn, int64_t nout, int64_t up_off, bool& valid) {
    if constexpr (GU) {
        const int wn = c / TN, j = (c / 32) % 2, l = c & 31;
        const int64_t o = (int64_t)tn * (bn / 2) + 32 * wn + l;
        valid = o < nout;
        return (valid ? o : 0) + (j ? up_off : 0);
    } else {
        const int64_t r = (int64_t)tn * bn + c;
        valid = r < nout;
        return valid ? r : 0;
    }
}

template <int WM, int WN, int MT, int NT, int RS, bool AFF, bool GU, typename YT, bool SPLIT>
__global__ __launch_bounds__(512) void k_gemm_fq(const uint8_t* __restrict__ Wq, const bf16_t* __restrict__ X,
                                                void* __restrict__ Yv, int M, int K, int64_t nout, int64_t up_off,
                                                int64_t ldy, int kps, int tiles_n, int tiles_m) {
    static_assert(WM * WN == 8, "8 waves");
    static_assert(!GU || NT == 2, "gate/up: a gate tile and an up tile per wave");
    constexpr int TM = 32 * MT, TN = 32 * NT;
    constexpr int BM = WM * TM, BN = WN * TN;
    static_assert(2 * BN <= 512 && BN % 64 == 0, "conversion split: two lanes per weight row");
    constexpr int RAWB = BN * 64 + BN * 16;  // nibble pieces + header dwords per raw slot (one quad)
    __shared__ __attribute__((aligned(16))) bf16_t Xs[3][BM * FQ_BK];
    __shared__ __attribute__((aligned(16))) bf16_t Ws[2][BN * FQ_BK];
    __shared__ __attribute__((aligned(16))) uint8_t Wr[RS][RAWB];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;
    int tn, tm, tz;
    fq_tile(tiles_n, tiles_m, tn, tm, tz);
    const int m0 = tm * BM;
    const int nsb = K >> 8;
    const int T = K / FQ_BK;
    const int t0 = tz * kps;
    const int t1 = t0 + kps < T ? t0 + kps : T;
    const int NS = t1 > t0 ? t1 - t0 : 0;

    // ---- copy roles.  Waves 0..3 copy x, waves 4..7 the raw weight tiles:
    // a wave's vector-memory counter completes in issue order, so an x copy
    // issued behind a raw copy that goes to HBM would count as pending until
    // that raw copy lands, and the raw tiles' latency would reach every step.
    const bool xw = wave < 4;
    const int rw = xw ? wave : wave - 4;
    constexpr int XC = BM / 64;         // x copies per x wave per step (BM / 4 rows)
    constexpr int RR = BN / 4;          // raw rows per raw wave
    constexpr int NC = RR / 16;         // nibble copies per raw wave per quad (16 rows x 64 B)
    constexpr int HC = (RR + 63) / 64;  // header copies per raw wave per quad (RR lanes of 16 B)
    constexpr int OFFN = XC > NC + HC ? XC : NC + HC;
    static_assert(RR % 16 == 0 && XC >= 1, "copy split");
    uint32_t off[OFFN];
    if (xw) {
        // lane -> row 16 i + lane / 4 of the wave's rows, LDS slot lane % 4,
        // which holds chunk fq_slot(row, slot); chunk c is columns +8 (c & 1) + 32 (c >> 1)
#pragma unroll
        for (int i = 0; i < OFFN; ++i) {
            const int r = rw * (BM / 4) + 16 * (i < XC ? i : 0) + (lane >> 2);
            int m = m0 + r;
            if (m >= M) m = M - 1;
            const int c = fq_slot(r, lane & 3);
            off[i] = (uint32_t)(((int64_t)m * K + 8 * (c & 1) + 32 * (c >> 1)) * 2);
        }
    } else {
        // nibble copy i: lane -> row rw * RR + 16 i + lane / 4, piece lane & 3
        // (the row's 64 B of the quad); header copy j: lane -> header lane
        // hl = 64 j + lane < RR: the row quad (rw * RR + 4 (hl / 4)) / 4, part
        // hl & 3 (16 B = its 4 rows' dword)
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            bool v;
            const int64_t nrow = fq_row<GU, TN>(rw * RR + 16 * i + (lane >> 2), tn, BN, nout, up_off, v);
            off[i] = (uint32_t)(q4k_group(nrow, nsb) + (nrow & 3) * (int64_t)nsb * 128 + 16 * (lane & 3));
        }
#pragma unroll
        for (int j = 0; j < HC; ++j) {
            bool v;
            const int hl = 64 * j + lane < RR ? 64 * j + lane : RR - 1;
            const int64_t hrow = fq_row<GU, TN>(rw * RR + (hl & ~3), tn, BN, nout, up_off, v);
            off[NC + j] = (uint32_t)(q4k_group(hrow, nsb) + (int64_t)nsb * 512 + 16 * (hl & 3));
        }
#pragma unroll
        for (int i = NC + HC; i < OFFN; ++i) off[i] = off[0];
    }
    const uint32_t xl = fq_lds(&Xs[0][0]) + rw * (BM / 4) * FQ_BK * 2;
    const uint32_t rl = fq_lds(&Wr[0][0]);
    auto copy_x = [&](int t) {
        if (!xw) return;
        const int s = t >> 3, h = (t >> 2) & 1, p = t & 3;
        const bf16_t* base = X + 256 * s + 64 * p + 16 * h;
#pragma unroll
        for (int i = 0; i < XC; ++i) fq_dma16(xl + (t % 3) * (BM * FQ_BK * 2) + i * 1024, base, off[i]);
    };
    // the raw tile of quad q (steps 4q .. 4q + 3)
    auto copy_raw = [&](int q) {
        if (xw) return;
        const int s = q >> 1, h = q & 1;
        const uint32_t l = rl + (q % RS) * RAWB;
#pragma unroll
        for (int i = 0; i < NC; ++i) fq_dma16(l + (rw * RR + 16 * i) * 64, Wq + (int64_t)h * nsb * 64 + 64 * s, off[i]);
#pragma unroll
        for (int j = 0; j < HC; ++j)
            if (64 * j + 64 <= RR || 64 * j + lane < RR) fq_dma16(l + BN * 64 + (rw * RR + 64 * j) * 16, Wq + 64 * s, off[NC + j]);
    };

    // ---- conversion: two lanes per weight row.  Unit u = (wave, lane) of the
    // block's 512 lanes, taken modulo 2 BN (lanes past 2 BN redo a unit and
    // store identical data to the same place: no branch splits the step): row
    // (u / 2), half u & 1 = bytes 8 half .. 8 half + 7 of the step's 16-B piece,
    // i.e. 8 low nibbles (k-slot chunk half) and 8 high (chunk 2 + half).
    const int cu = (wave * 64 + lane) % (2 * BN);
    const int crow = cu >> 1, chalf = cu & 1;
    bool cvalid;
    (void)fq_row<GU, TN>(crow, tn, BN, nout, up_off, cvalid);
    // raw tile of step t -> the lane's 8 bf16 pairs (low chunk, high chunk)
    auto convert = [&](int t, uint32_t (&o)[8]) {
        const uint8_t* raw = &Wr[(t >> 2) % RS][0];
        const int p = t & 3;
        const uint2 nib = *reinterpret_cast<const uint2*>(raw + crow * 64 + p * 16 + chalf * 8);
        // header dwords of row crow: [quad][p'][r] in the raw slot
        const uint32_t* hq = reinterpret_cast<const uint32_t*>(raw + BN * 64) + (crow >> 2) * 16 + (crow & 3);
        float dl, ml, dh, mh;
        if constexpr (AFF) {
            const uint32_t hw = hq[4 * p];
            dl = dh = aff_scale(hw);
            ml = mh = -aff_bias(hw);
        } else {
            const uint4 hd = make_uint4(hq[0], hq[4], hq[8], hq[12]);
            const uint32_t hw = p == 0 ? hd.x : (p == 1 ? hd.y : (p == 2 ? hd.z : hd.w));
            const float d = q4k_hdr_d(hd), dmin = q4k_hdr_dmin(hd);
            dl = d * (float)(hw & 63u);
            ml = dmin * (float)((hw >> 6) & 63u);
            dh = d * (float)((hw >> 12) & 63u);
            mh = dmin * (float)((hw >> 18) & 63u);
        }
        if (!cvalid) dl = ml = dh = mh = 0.0f;
        const uint32_t q[2] = {nib.x, nib.y};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t lo = q[i] & 0x0F0F0F0Fu, hi = (q[i] >> 4) & 0x0F0F0F0Fu;
            o[2 * i] = pack_bf16x2(__builtin_fmaf(dl, ubyte_f32<0>(lo), -ml), __builtin_fmaf(dl, ubyte_f32<1>(lo), -ml));
            o[2 * i + 1] =
                pack_bf16x2(__builtin_fmaf(dl, ubyte_f32<2>(lo), -ml), __builtin_fmaf(dl, ubyte_f32<3>(lo), -ml));
            o[4 + 2 * i] =
                pack_bf16x2(__builtin_fmaf(dh, ubyte_f32<0>(hi), -mh), __builtin_fmaf(dh, ubyte_f32<1>(hi), -mh));
            o[4 + 2 * i + 1] =
                pack_bf16x2(__builtin_fmaf(dh, ubyte_f32<2>(hi), -mh), __builtin_fmaf(dh, ubyte_f32<3>(hi), -mh));
        }
    };
    auto store_w = [&](int t, const uint32_t (&o)[8]) {
        bf16_t* wt = &Ws[t & 1][0];
        *reinterpret_cast<uint4*>(wt + fq_swz(crow, chalf)) = make_uint4(o[0], o[1], o[2], o[3]);
        *reinterpret_cast<uint4*>(wt + fq_swz(crow, 2 + chalf)) = make_uint4(o[4], o[5], o[6], o[7]);
    };

    const int lr = lane & 31, lh = lane >> 5;
    f32x16_t acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    // copies: x(t) two steps ahead (3 slots) by the x waves; the raw tile of
    // quad q + RS - 1 at the top of step 4q by the raw waves (RS slots: the
    // quad's data is first converted during step 4 (q + RS - 1) - 1, 4 RS - 5
    // steps later).  Splits start on a quad.  Each wave waits only on its own
    // stream: x(t) for the x waves, the raw quad of step t + 1 for the raw waves.
    const int q0 = t0 >> 2, qlast = (t1 - 1) >> 2;
    const int pre = qlast - q0 + 1 < RS - 1 ? qlast - q0 + 1 : RS - 1;  // quads copied in the prologue
    auto raw_at = [&](int i) {  // step i copies the raw tile of quad Q(t) + RS - 1
        const int t = t0 + i;
        return (t & 3) == 0 && (t >> 2) + RS - 1 <= qlast;
    };
    // raw-wave wait before step i (or the prologue, i = -1): the quads copied
    // so far are q0 .. q0 + n - 1; the one needed is that of step t + 1
    auto raw_wait = [&](int i) {
        int n = pre + (i >= 0 ? (i + 3) / 4 : 0);
        if (n > qlast - q0 + 1) n = qlast - q0 + 1;
        const int need = i >= 0 ? ((t0 + i + 1) >> 2) - q0 : 0;
        const int after = n - 1 - need;  // quads copied after the needed one
        if (i >= 0 && t0 + i + 1 >= t1) fq_wait_vm<0>();
        else if (after <= 0) fq_wait_vm<0>();
        else if (after == 1) fq_wait_vm<NC + HC>();
        else fq_wait_vm<2 * (NC + HC)>();
    };
    static_assert(RS <= 3, "raw_wait covers up to two quads in flight");
    if (NS > 0) {
#pragma unroll
        for (int q = 0; q < RS - 1; ++q)
            if (q < pre) copy_raw(q0 + q);
        copy_x(t0);
        if (NS > 1) copy_x(t0 + 1);
        if (!xw) raw_wait(-1);
        __syncthreads();
        uint32_t o[8];
        convert(t0, o);
        store_w(t0, o);
    }
    for (int i = 0; i < NS; ++i) {
        const int t = t0 + i;
        if (xw) {
            if (i + 1 < NS) fq_wait_vm<XC>();  // x(t + 1) may stay in flight
            else fq_wait_vm<0>();
        } else {
            raw_wait(i);
        }
        __syncthreads();  // x(t), raw(t + 1) and the converted W(t) visible to all
        if (i + 2 < NS) copy_x(t + 2);
        if (raw_at(i)) copy_raw((t >> 2) + RS - 1);
        const bf16_t* xs = &Xs[t % 3][0];
        const bf16_t* ws = &Ws[t & 1][0];
        // step t + 1's weights are converted while step t's MFMAs run (at the
        // last step the conversion reads a stale raw slot into the idle W
        // buffer, which nothing reads: no branch splits the step)
        uint32_t o[8];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int ch = 2 * kk + lh;
            bf16x8_t a[MT], b[NT];
#pragma unroll
            for (int ii = 0; ii < MT; ++ii)
                a[ii] = *reinterpret_cast<const bf16x8_t*>(xs + fq_swz(wm * TM + 32 * ii + lr, ch));
#pragma unroll
            for (int j = 0; j < NT; ++j)
                b[j] = *reinterpret_cast<const bf16x8_t*>(ws + fq_swz(wn * TN + 32 * j + lr, ch));
            if (kk == 0) convert(t + 1, o);
#pragma unroll
            for (int ii = 0; ii < MT; ++ii)
#pragma unroll
                for (int j = 0; j < NT; ++j) acc[ii][j] = fq_mfma(a[ii], b[j], acc[ii][j]);
        }
        store_w(t + 1, o);
        // issue order: the conversion's VALU spread between the step's MFMAs
        // (one MFMA, then up to FQ_VPM VALU), so it runs in the MFMA shadow
#pragma unroll
        for (int r = 0; r < 2 * MT * NT; ++r) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, FQ_VPM, 0);
        }
    }

    fq_wait_vm<0>();  // no copy may land in LDS after the block

    // epilogue: lane holds column lr of each 32 x 32 tile, rows 8 (e / 4) + 4 (lane / 32) + e % 4
#pragma unroll
    for (int ii = 0; ii < MT; ++ii)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int m = m0 + wm * TM + 32 * ii + 8 * (e >> 2) + 4 * lh + (e & 3);
            if (m >= M) continue;
            if constexpr (GU) {
                const int64_t o = (int64_t)tn * (BN / 2) + 32 * wn + lr;
                if (o >= nout) continue;
                if constexpr (SPLIT) {
                    float* P = static_cast<float*>(Yv) + (int64_t)tz * M * ldy;
                    P[(int64_t)m * ldy + o] = acc[ii][0][e];
                    P[(int64_t)m * ldy + up_off + o] = acc[ii][1][e];
                } else {
                    store_y<YT>(static_cast<YT*>(Yv) + (int64_t)m * ldy + o, silu_mul(acc[ii][0][e], acc[ii][1][e]));
                }
            } else {
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    const int64_t n = (int64_t)tn * BN + wn * TN + 32 * j + lr;
                    if (n >= nout) continue;
                    if constexpr (SPLIT)
                        (static_cast<float*>(Yv) + (int64_t)tz * M * ldy)[(int64_t)m * ldy + n] = acc[ii][j][e];
                    else
                        store_y<YT>(static_cast<YT*>(Yv) + (int64_t)m * ldy + n, acc[ii][j][e]);
                }
            }
        }
}

template <int WM, int WN, int MT, int NT, int RS, bool AFF, bool GU, typename YT>
hipError_t fq_launch(const FqPlan& p, const uint8_t* wq, const bf16_t* x, void* y, float* ws, int M, int K,
                     int64_t nout, int64_t up_off, int64_t n_rows, hipStream_t s) {
    const unsigned nb = (unsigned)(p.tiles_n * p.tiles_m * p.splits);
    if (p.splits == 1) {
        hipLaunchKernelGGL((k_gemm_fq<WM, WN, MT, NT, RS, AFF, GU, YT, false>), dim3(nb), dim3(512), 0, s, wq, x, y, M, K,
                           nout, up_off, nout, p.kps, p.tiles_n, p.tiles_m);
        return hipGetLastError();
    }
    hipLaunchKernelGGL((k_gemm_fq<WM, WN, MT, NT, RS, AFF, GU, float, true>), dim3(nb), dim3(512), 0, s, wq, x,
                       (void*)ws, M, K, nout, up_off, n_rows, p.kps, p.tiles_n, p.tiles_m);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_split_reduce(ws, y, std::is_same<YT, float>::value, GU, M, nout, up_off, n_rows, p.splits, s);
}

template <bool AFF, bool GU, typename YT>
hipError_t fq_geom(const FqPlan& p, const uint8_t* wq, const bf16_t* x, void* y, float* ws, int M, int K,
                   int64_t nout, int64_t up_off, int64_t n_rows, hipStream_t s) {
    if constexpr (GU) {
        // 256 x 256 tiles (128 outputs): 2 x 4 waves of 128 x (32 gate + 32 up)
        return fq_launch<2, 4, 4, 2, 3, AFF, true, YT>(p, wq, x, y, ws, M, K, nout, up_off, n_rows, s);
    } else {
        // raw rings: 2 quads for the 512 x 192 tile (150 KB of LDS), 3 for the others
        if (p.geom == 3) return fq_launch<4, 2, 4, 3, 2, AFF, false, YT>(p, wq, x, y, ws, M, K, nout, up_off, n_rows, s);
        if (p.geom == 1) return fq_launch<2, 4, 4, 2, 3, AFF, false, YT>(p, wq, x, y, ws, M, K, nout, up_off, n_rows, s);
        return fq_launch<2, 4, 2, 2, 3, AFF, false, YT>(p, wq, x, y, ws, M, K, nout, up_off, n_rows, s);
    }
}

}  // namespace

// geometries: 1 = 256 x 256, 2 = 128 x 256, 3 = 512 x 192; gate/up always
// 256 x 256 (128 outputs)
static void fq_dims(int geom, bool gu, int& bm, int& bn) {
    if (geom == 3 && !gu) {
        bm = 512;
        bn = 192;
    } else if (gu || geom == 1) {
        bm = 256;
        bn = 256;
    } else {
        bm = 128;
        bn = 256;
    }
}

bool gemm_fq_supported(int64_t M, int64_t N_rows, int64_t K, bool gu) {
    // the row-quad plane (N padded to 4 rows) and x below 4 GiB for the
    // 32-bit copy offsets; whole superblocks; gate/up: the up half starts on
    // a row quad (the header copies take 4 rows of one quad)
    const uint64_t wbytes = (uint64_t)((N_rows + 3) / 4) * (uint64_t)(K / 256) * 576;
    return M >= 1 && N_rows >= 1 && K >= 256 && K % 256 == 0 && (uint64_t)M * (uint64_t)K * 2 < (1ull << 32) &&
           wbytes < (1ull << 32) && M < (1 << 30) && (!gu || (N_rows % 8 == 0));
}

static int fq_env(const char* name, int dflt) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

// Geometry and K split.  Modeled time = rounds of resident blocks (one block
// of 8 waves per CU) x steps per block x step time, plus, with splits, the
// f32 partials' round trip (written once, read once by the reduce: 8 B per
// output per split at 5 TB/s) and the reduce launch.  A step costs its MFMA
// cycles at 65 % of the 2.05 GHz rate sustained under MFMA load, and no less
// than 0.55 us (one barrier, the LDS operand reads and the dependent
// conversion of the next step's weights).  Splits start on a superblock (8
// steps).  THQ_FQ_GEOM / THQ_FQ_SPLITS force a choice (tuning).
FqPlan plan_gemm_fq(int64_t M, int64_t N_rows, int64_t K, bool gu, int cus) {
    FqPlan p;
    if (cus < 1) cus = 256;
    const int T = (int)(K / FQ_BK);
    const int fg = fq_env("THQ_FQ_GEOM", -1), fs = fq_env("THQ_FQ_SPLITS", 0);
    double best = -1.0;
    for (int g = 1; g < 4; ++g) {
        if ((gu && g != 1) || (fg >= 0 && g != fg)) continue;
        int bm, bn;
        fq_dims(g, gu, bm, bn);
        const int64_t tm = (M + bm - 1) / bm, tn = (N_rows + bn - 1) / bn;
        const double mfma_cycles = (double)bm * bn * FQ_BK * 2.0 / 4096.0;  // per CU per step (4 SIMDs x 1024 flop/clk)
        double tstep = mfma_cycles / (2.05e3 * 0.65);                        // us
        if (tstep < 0.55) tstep = 0.55;
        for (int sp = 1; sp <= 16; ++sp) {
            if (fs > 0 && sp != fs) continue;
            int kps = (T + sp - 1) / sp;
            kps = (kps + 7) / 8 * 8;
            if (kps > T) kps = T;
            const int splits = (T + kps - 1) / kps;
            if (splits != sp && fs <= 0) continue;  // the same plan as a smaller count
            const int64_t blocks = tm * tn * splits;
            const int64_t rounds = (blocks + cus - 1) / cus;
            double t = (double)rounds * kps * tstep;
            if (splits > 1) t += (double)splits * (double)M * (double)N_rows * 8.0 / 5.0e6 + 3.0;
            if (best < 0.0 || t < best) {
                best = t;
                p.geom = g;
                p.tiles_m = (int)tm;
                p.tiles_n = (int)tn;
                p.kps = kps;
                p.splits = splits;
            }
        }
    }
    p.workspace_bytes = p.splits > 1 ? (size_t)p.splits * (size_t)M * (size_t)N_rows * sizeof(float) : 0;
    return p;
}

hipError_t launch_gemm_fq(const FqPlan& p, bool aff, const uint8_t* wq, const void* x, void* y, bool yf32, bool gu,
                          int M, int64_t N_rows, int K, float* ws, hipStream_t s) {
    const bf16_t* xb = static_cast<const bf16_t*>(x);
    const int64_t nout = gu ? N_rows / 2 : N_rows, up_off = gu ? N_rows / 2 : 0;
    if (aff) {
        if (gu) return yf32 ? fq_geom<true, true, float>(p, wq, xb, y, ws, M, K, nout, up_off, N_rows, s)
                            : fq_geom<true, true, bf16_t>(p, wq, xb, y, ws, M, K, nout, up_off, N_rows, s);
        return yf32 ? fq_geom<true, false, float>(p, wq, xb, y, ws, M, K, nout, up_off, N_rows, s)
                    : fq_geom<true, false, bf16_t>(p, wq, xb, y, ws, M, K, nout, up_off, N_rows, s);
    }
    if (gu) return yf32 ? fq_geom<false, true, float>(p, wq, xb, y, ws, M, K, nout, up_off, N_rows, s)
                        : fq_geom<false, true, bf16_t>(p, wq, xb, y, ws, M, K, nout, up_off, N_rows, s);
    return yf32 ? fq_geom<false, false, float>(p, wq, xb, y, ws, M, K, nout, up_off, N_rows, s)
                : fq_geom<false, false, bf16_t>(p, wq, xb, y, ws, M, K, nout, up_off, N_rows, s);
}

}  // namespace thq
