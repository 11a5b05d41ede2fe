// k_gemm_rq.hip — prefill GEMM from 1024 rows (any M with THQ_GEMM_RQ=1):
// y[M, N] = x[M, K] (bf16) . W[N, K]^T with W in Q4_K or MLX affine 4-bit
// row quads, each wave's weight rows dequantized in registers straight into
// MFMA operands.
//
// Role: the m > 8 projections of the reference (AffineQpf, routed by
// pf_route / pf_policy, engine/src/quant_kernel.rs:5117-5300); fused gate/up
// with the silu(gate)*up epilogue (engine/src/quant_kernel.rs:2922-2926).
//
// Tiling: 8 waves per block, one block per CU.  Each wave owns 32 weight
// rows and every M row of the block (wave tile BM x 32, block tile BM x 256,
// BM = 128 or 256), so each weight is converted once per block, by the one
// wave that multiplies it, into the B operand of its v_mfma_f32_32x32x16_bf16
// (about 150 VALU per 4 * BM/32 MFMAs).  Without the copies the K loop runs
// at the MFMA rate (12288 x 4096 at M = 256 on 48 CUs: 1.03 us per 64-wide K
// step, 2048 MFMA cycles per SIMD); the direct-to-LDS copies of x (from L2)
// and of the weights (from HBM) add about 0.3 us each per step, neither
// hidden by deeper rings nor by separate issuing waves: that is where this
// tile stands against the others (below 1024 rows the tile GEMM, whose
// smaller blocks fill the CUs, is as fast or faster).
//
// Data movement (all direct-to-LDS copies, global_load_lds_dwordx4):
//   x ring   2 (BM = 256) or 3 slots of the BM x 64 bf16 x tile (rows of
//            128 B, 16-B chunk c of row r at slot c ^ ((r >> 1) & 7)),
//            copied by waves 0..3 one or two K steps ahead
//   W ring   7 or 9 slots, copied by waves 4..7 six or eight K steps ahead:
//            per step the block's 256 rows x 32 nibble bytes (the step's two
//            16-B pieces of each row) and the 64-B header run of each row
//            quad's superblock
//   Each copying wave waits only on its own stream; one block barrier per K
//   step publishes both.
// Operand order within a 64-wide K step: lane half h of a wave holds nibble
// piece h of its row (bytes 16h .. 16h+15: low nibbles = weights 16h .. +15,
// high = 32 + 16h .. +15).  MFMA k-group kk takes from each half the 8
// weights of one dword pair (kk = 0: low nibbles of bytes 0..7, 1: low of
// 8..15, 2: high of 0..7, 3: high of 8..15), and the A fragment reads x
// chunk {0, 1, 4, 5}[kk] + 2h: the same K set, in a permuted order, on both
// sides.
// Weight values: bf16(fma(s, 128 + q, -(128 s + m))) with s = d * sc and
// m = dmin * mn (Q4_K) or s = scale, 128 s - bias (affine), the values of
// k_gemm_dma's rounded tiles.
// Grid: fewer tiles than CUs: K is split into equal ranges; more: whole
// rounds of tiles over all of K, then the last partial round (at most half
// the CUs) in halves.  The split tiles meet in the last block to arrive
// (the ordering argument is at the ticket below), which sums the splits in
// split order: deterministic.
// Offsets are 32-bit: the router sends x or weights of 4 GiB and more
// elsewhere.
#include "thq_dev.hpp"
#include "thq_kernels.hpp"

namespace thq {
namespace {

constexpr int RQ_BK = 64;                             // K per step
constexpr int RQ_NW = 8;                              // waves per block
constexpr int RQ_BN = 32 * RQ_NW;                     // weight rows per block (32 per wave)
constexpr int RQ_NIB = RQ_BN * 32;                    // nibble bytes per step
constexpr int RQ_WSLOT = RQ_NIB + (RQ_BN / 4) * 64;   // + 64-B header run per row quad (12 KB)
// ring slots: x (from L2) one step ahead, weights (from HBM) six or eight
template <int BM> struct RqRing {
    static constexpr int NXS = BM == 256 ? 2 : 3, NWS = BM == 256 ? 7 : 9;
    static constexpr int LX = NXS - 1, LW = NWS - 1;
    static_assert(LW >= 2, "the next step's weights are copied before this step");
};

__device__ __forceinline__ uint32_t rq_lds(const void* p) {
    return (uint32_t)(size_t)(__attribute__((address_space(3))) const void*)p;
}
// 16 bytes per lane from base + voff to LDS at m0 + 16 * lane.  Inline asm:
// the compiler's own waits would put a vmcnt(0) before every LDS read that
// follows a direct-to-LDS load.
__device__ __forceinline__ void rq_dma16(uint32_t lds, const void* base, uint32_t voff) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"{m0}"(lds), "v"(voff), "s"(base) : "memory");
}
template <int N>
__device__ __forceinline__ void rq_wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ int rq_swz(int r, int c) { return r * RQ_BK + ((c ^ ((r >> 1) & 7)) << 3); }
// 16-B agent-scope (sc1) vector store / load of the split partials: performed
// at the level where every XCD's accesses are coherent.  The loads' data is
// valid only after an s_waitcnt vmcnt that names the destination registers
// (rq_wait_vm4 below), since the compiler does not track these loads.
__device__ __forceinline__ void rq_st16(float* p, const f32x4_t& v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void rq_ld16(f32x4_t& v, const float* p) {
    asm volatile("global_load_dwordx4 %0, %1, off sc1" : "=v"(v) : "v"(p) : "memory");
}
__device__ __forceinline__ void rq_wait_vm4(f32x4_t (&v)[4][4]) {
    asm volatile("s_waitcnt vmcnt(0)"
                 : "+v"(v[0][0]), "+v"(v[0][1]), "+v"(v[0][2]), "+v"(v[0][3]), "+v"(v[1][0]), "+v"(v[1][1]),
                   "+v"(v[1][2]), "+v"(v[1][3]), "+v"(v[2][0]), "+v"(v[2][1]), "+v"(v[2][2]), "+v"(v[2][3]),
                   "+v"(v[3][0]), "+v"(v[3][1]), "+v"(v[3][2]), "+v"(v[3][3])::"memory");
}

// tile row j (0..RQ_BN-1) of output tile tn -> weight row; gate/up: each wave's
// 32 rows are 16 gate rows then the 16 up rows of the same outputs
template <bool GU>
__device__ __forceinline__ int64_t rq_row(int tn, int j, int64_t nout, int64_t up_off, bool& valid) {
    if (GU) {
        const int64_t o = (int64_t)tn * (RQ_BN / 2) + 16 * (j >> 5) + (j & 15);
        valid = o < nout;
        return o + ((j & 16) ? up_off : 0);
    }
    const int64_t n = (int64_t)tn * RQ_BN + j;
    valid = n < nout;
    return n;
}

// block b of a range of nb blocks that starts on a multiple of 8 -> its
// index within the range such that XCD x = b & 7 runs a contiguous part
__device__ __forceinline__ int rq_xcd_index(int b, int nb) {
    const int q = (nb + 7) >> 3, tall = (nb & 7) ? (nb & 7) : 8;
    const int xcd = b & 7, local = b >> 3;
    return xcd < tall ? xcd * q + local : tall * q + (xcd - tall) * (q - 1) + local;
}
// block -> (column tile, row tile, split, splits of its tile).  The first
// `whole` blocks compute tiles 0 .. whole-1 over all of K; the remaining
// tiles are split in `splits` K ranges each (one block per range).  Tiles
// are numbered column tiles fastest, so an XCD's blocks share x rows.
__device__ __forceinline__ void rq_tile(int tiles_n, int whole, int splits, int& tn, int& tm, int& z, int& ns) {
    const int nb = gridDim.x, b = blockIdx.x;
    int tile;
    if (b < whole) {
        tile = rq_xcd_index(b, whole);
        z = 0;
        ns = 1;
    } else {
        const int L = rq_xcd_index(b - whole, nb - whole);
        tile = whole + L / splits;
        z = L % splits;
        ns = splits;
    }
    tn = tile % tiles_n;
    tm = tile / tiles_n;
}

// bytes 0..3 of v (codes 0..15) -> bf16(fma(s, 128 + q, -c)) as two dwords
__device__ __forceinline__ void rq_cvt4(uint32_t v, float s, float c, uint32_t& lo, uint32_t& hi) {
    const float f0 = __uint_as_float(__builtin_amdgcn_perm(0x43434343u, v, 0x04000c0cu));
    const float f1 = __uint_as_float(__builtin_amdgcn_perm(0x43434343u, v, 0x04010c0cu));
    const float f2 = __uint_as_float(__builtin_amdgcn_perm(0x43434343u, v, 0x04020c0cu));
    const float f3 = __uint_as_float(__builtin_amdgcn_perm(0x43434343u, v, 0x04030c0cu));
    lo = pack_bf16x2(__builtin_fmaf(s, f0, -c), __builtin_fmaf(s, f1, -c));
    hi = pack_bf16x2(__builtin_fmaf(s, f2, -c), __builtin_fmaf(s, f3, -c));
}
// the 8 weights of dwords (a, b), nibble `hi` (0 low, 1 high), as an MFMA operand
__device__ __forceinline__ bf16x8_t rq_b(uint32_t a, uint32_t b, int hi, float s, float c) {
    const uint32_t qa = (hi ? a >> 4 : a) & 0x0F0F0F0Fu, qb = (hi ? b >> 4 : b) & 0x0F0F0F0Fu;
    uint4 o;
    rq_cvt4(qa, s, c, o.x, o.y);
    rq_cvt4(qb, s, c, o.z, o.w);
    return as_bf16x8(o);
}
__device__ __forceinline__ f32x16_t rq_mfma(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// one block of 8 waves per CU: two waves per SIMD, 256 registers each
template <int QT, int BM, bool GU, typename YT>
__global__ __launch_bounds__(64 * RQ_NW) __attribute__((amdgpu_waves_per_eu(2))) void k_gemm_rq(const uint8_t* __restrict__ Wq, const bf16_t* __restrict__ X,
                                                YT* __restrict__ Y, float* __restrict__ P, uint32_t* __restrict__ cnt,
                                                int M, int K, int64_t nout, int64_t up_off, int tiles_n, int whole,
                                                int splits, int kps) {
    constexpr int MT = BM / 32;  // 32-row MFMA tiles per wave (the wave covers all BM rows)
    constexpr int NXS = RqRing<BM>::NXS, NWS = RqRing<BM>::NWS, LX = RqRing<BM>::LX, LW = RqRing<BM>::LW;
    // copy roles: waves 0 .. 3 copy x, waves 4 .. 7 the weights of two waves
    // each, so that each wave's in-order vmcnt covers one stream and the
    // weights' deeper ring really buys latency
    constexpr int XW = RQ_NW / 2;
    constexpr int XI = BM / (8 * XW);  // x copies per x wave per step: BM rows x 8 chunks / 4 waves / 64 lanes
    __shared__ __attribute__((aligned(16))) bf16_t Xs[NXS][BM * RQ_BK];
    __shared__ __attribute__((aligned(16))) uint8_t Wr[NWS][RQ_WSLOT];
    __shared__ uint32_t last_split;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 31, hf = lane >> 5;
    int tn, tm, z, ns;
    rq_tile(tiles_n, whole, splits, tn, tm, z, ns);
    const int T = K / RQ_BK, nsb = K >> 8;
    const int k0 = ns > 1 ? z * kps : 0;
    const int n = ns > 1 ? (k0 + kps < T ? k0 + kps : T) - k0 : T;  // steps of this block (>= 1: no empty split)
    const int m0 = tm * BM;

    // ---- copy descriptors (x waves: xoff; weight waves: noff, hoff)
    const bool xrole = wave < XW;
    uint32_t xoff[XI];
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        // lane -> row r, LDS slot lane & 7, which holds chunk (lane & 7) ^ ((r >> 1) & 7)
        const int r = (wave % XW) * (BM / XW) + 8 * i + (lane >> 3);
        const int c = (lane & 7) ^ ((r >> 1) & 7);
        const int m = m0 + r < M ? m0 + r : M - 1;
        xoff[i] = (uint32_t)(((int64_t)m * K + 8 * c) * 2);
    }
    const uint32_t xl = rq_lds(&Xs[0][0]) + (wave % XW) * (BM / XW) * 128;
    const int ww = wave % XW;  // weight wave: the rows of waves 2 ww and 2 ww + 1
    uint32_t noff[2], hoff;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        // nibbles: 16-B position 64 * w + lane of the step slot (w = 2 ww + k)
        // = tile row j, piece (lane & 1) ^ ((j >> 3) & 1) (two rows' pieces per
        // bank row)
        const int j = 32 * (2 * ww + k) + (lane >> 1);
        const int h = (lane & 1) ^ ((j >> 3) & 1);
        bool v;
        int64_t row = rq_row<GU>(tn, j, nout, up_off, v);
        if (!v) row = 0;
        noff[k] = (uint32_t)q4k_piece(row, nsb, 0, h, 0);
    }
    {
        // headers: row quad 16 ww + lane / 4, part lane % 4
        const int qd = 16 * ww + (lane >> 2);
        bool v;
        int64_t r0 = rq_row<GU>(tn, 4 * qd, nout, up_off, v);
        if (!v) r0 = 0;
        hoff = (uint32_t)(q4k_group(r0, nsb) + (int64_t)nsb * 512 + (lane & 3) * 16);
    }
    const uint32_t nl = rq_lds(&Wr[0][0]) + ww * 2048;
    const uint32_t hl = rq_lds(&Wr[0][0]) + RQ_NIB + ww * 1024;
    // kit and slot are uniform; readfirstlane keeps the base addresses in
    // SGPRs, as the copy instruction requires.  copy(kit, xslot, wslot):
    // this wave's share of x or of the weights of K step kit
    auto xcopy = [&](int kit, int slot) {
        kit = __builtin_amdgcn_readfirstlane(kit);
        slot = __builtin_amdgcn_readfirstlane(slot);
        const bf16_t* base = X + kit * RQ_BK;
#pragma unroll
        for (int i = 0; i < XI; ++i) rq_dma16(xl + slot * (BM * RQ_BK * 2) + i * 1024, base, xoff[i]);
    };
    auto wcopy = [&](int kit, int slot) {
        kit = __builtin_amdgcn_readfirstlane(kit);
        slot = __builtin_amdgcn_readfirstlane(slot);
        rq_dma16(nl + slot * RQ_WSLOT, Wq + kit * 16, noff[0]);
        rq_dma16(nl + slot * RQ_WSLOT + 1024, Wq + kit * 16, noff[1]);
        rq_dma16(hl + slot * RQ_WSLOT, Wq + (kit >> 2) * 64, hoff);
    };

    // ---- this lane's weight row and its reads from a W slot
    const int jr = 32 * wave + lr;
    bool rvalid;
    (void)rq_row<GU>(tn, jr, nout, up_off, rvalid);
    const int npos = (2 * jr + (hf ^ ((jr >> 3) & 1))) * 16;            // its nibble piece
    const int hpos = RQ_NIB + (jr >> 2) * 64 + (jr & 3) * 4;            // its header dword of part 0
    struct Wv {
        uint4 q;                // nibble piece
        float s0, c0, s1, c1;   // scale / offset of the step's low and high nibbles
    };
    auto wread = [&](int slot, int kit) {
        Wv r;
        const uint8_t* w = &Wr[slot][0];
        r.q = *reinterpret_cast<const uint4*>(w + npos);
        const int p = kit & 3;
        const uint32_t hp = *reinterpret_cast<const uint32_t*>(w + hpos + p * 16);
        if constexpr (QT == 13) {  // affine group of 64: w = scale * (128 + q) - (128 * scale - bias)
            const float sc = rvalid ? aff_scale(hp) : 0.0f, bi = rvalid ? aff_bias(hp) : 0.0f;
            r.s0 = r.s1 = sc;
            r.c0 = r.c1 = __builtin_fmaf(128.0f, sc, -bi);
        } else {
            const uint32_t h0 = *reinterpret_cast<const uint32_t*>(w + hpos);
            const uint32_t h1 = *reinterpret_cast<const uint32_t*>(w + hpos + 16);
            const uint32_t h2 = *reinterpret_cast<const uint32_t*>(w + hpos + 32);
            const uint32_t h3 = *reinterpret_cast<const uint32_t*>(w + hpos + 48);
            float d = q4k_hdr_d(make_uint4(h0, h1, h2, h3)), dm = q4k_hdr_dmin(make_uint4(h0, h1, h2, h3));
            if (!rvalid) d = dm = 0.0f;
            r.s0 = d * (float)(hp & 63u);
            r.c0 = __builtin_fmaf(128.0f, r.s0, dm * (float)((hp >> 6) & 63u));
            r.s1 = d * (float)((hp >> 12) & 63u);
            r.c1 = __builtin_fmaf(128.0f, r.s1, dm * (float)((hp >> 18) & 63u));
        }
        return r;
    };

    f32x16_t acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;

    // ---- prologue: weights of steps 0 .. LW-1 or x of steps 0 .. LX-1 (the
    // clamped copies past the block's last step land in slots no step reads)
    if (xrole) {
#pragma unroll
        for (int i = 0; i < LX; ++i) xcopy(k0 + (i < n ? i : n - 1), i);
    } else {
#pragma unroll
        for (int i = 0; i < LW; ++i) wcopy(k0 + (i < n ? i : n - 1), i);
    }

    Wv wv;
    bf16x8_t b0;
    for (int t = 0; t < n; ++t) {
        // x waves: x(t) has landed; weight waves: the weights of steps t and
        // t + 1.  After the barrier, for every wave, and every wave is past
        // step t - 1, whose slots the next copies refill
        if (xrole) rq_wait_vm<(LX - 1) * XI>();
        else rq_wait_vm<3 * (LW - 2)>();
        __syncthreads();
        if (xrole) {
            const int ux = t + LX;
            xcopy(k0 + (ux < n ? ux : n - 1), ux % NXS);
        } else {
            const int uw = t + LW;
            wcopy(k0 + (uw < n ? uw : n - 1), uw % NWS);
        }
        const int kit = k0 + t;
        if (t == 0) {
            wv = wread(0, kit);
            b0 = rq_b(wv.q.x, wv.q.y, 0, wv.s0, wv.c0);
        }
        const bf16_t* xs = &Xs[t % NXS][0];
        // A fragments of k-group kk (x chunk {0, 1, 4, 5}[kk] + 2 hf), read
        // one group ahead into two register sets; each group's MFMAs are
        // interleaved with the conversion of a later group's B operand
        bf16x8_t a0[MT], a1[MT];
        auto aread = [&](bf16x8_t* a, int ch) {
#pragma unroll
            for (int i = 0; i < MT; ++i) a[i] = *reinterpret_cast<const bf16x8_t*>(xs + rq_swz(32 * i + lr, ch + 2 * hf));
        };
        auto mfmas = [&](const bf16x8_t* a, const bf16x8_t& b) {
#pragma unroll
            for (int i = 0; i < MT; ++i) acc[i] = rq_mfma(a[i], b, acc[i]);
        };
        // VALU per MFMA in a group: a B conversion is ~24 VALU.  Full
        // scheduling barriers between the phases keep each group's fragment
        // reads one group ahead of its MFMAs (the scheduler otherwise sinks
        // them to their use, exposing the LDS latency in every group)
        constexpr int VPM = (24 + MT - 1) / MT;
        auto interleave = [&]() {
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
            }
        };
        aread(a0, 0);
        const bf16x8_t b1 = rq_b(wv.q.z, wv.q.w, 0, wv.s0, wv.c0);
        aread(a1, 1);
        __builtin_amdgcn_sched_barrier(0);
        // group 0, converting b2
        mfmas(a0, b0);
        const bf16x8_t b2 = rq_b(wv.q.x, wv.q.y, 1, wv.s1, wv.c1);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
        aread(a0, 4);
        __builtin_amdgcn_sched_barrier(0);
        // group 1, converting b3
        mfmas(a1, b1);
        const bf16x8_t b3 = rq_b(wv.q.z, wv.q.w, 1, wv.s1, wv.c1);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
        aread(a1, 5);
        __builtin_amdgcn_sched_barrier(0);
        // group 2, reading the next step's weights (they have landed; past
        // the last step this reads a slot of clamped copies, unused)
        mfmas(a0, b2);
        wv = wread((t + 1) % NWS, kit + 1);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
        // group 3, converting the next step's b0
        mfmas(a1, b3);
        b0 = rq_b(wv.q.x, wv.q.y, 0, wv.s0, wv.c0);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
    }
    rq_wait_vm<0>();  // no copy may land in LDS after the block

    // lane holds column lr of each 32 x 32 tile, rows 8 (e / 4) + 4 hf + e % 4
    auto store_tile = [&](int i, const float* v) {
        const int mi = m0 + 32 * i + 4 * hf;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int m = mi + 8 * (e >> 2) + (e & 3);
            if (GU) {
                // gate in lanes lr < 16, up of the same output 16 lanes up
                const float u = __shfl_xor(v[e], 16, 64);
                const int64_t o = (int64_t)tn * (RQ_BN / 2) + 16 * wave + lr;
                if (lr < 16 && m < M && o < nout) store_y<YT>(Y + (int64_t)m * nout + o, silu_mul(v[e], u));
            } else {
                const int64_t o = (int64_t)tn * RQ_BN + 32 * wave + lr;
                if (m < M && o < nout) store_y<YT>(Y + (int64_t)m * nout + o, v[e]);
            }
        }
    };
    if (ns == 1) {
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            float v[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] = acc[i][e];
            store_tile(i, v);
            asm volatile("" ::: "memory");  // one 32-row tile's stores at a time
        }
        return;
    }
    // split-K: this split's tile in lane order, 16 B per lane (elements
    // 4g .. 4g+3 of 32-row tile i of wave w at ((i * 4 + g) * 8 + w) * 64 +
    // lane, in 16-B units: every instruction covers 1 KB contiguous); the
    // last block to arrive sums all splits of the tile, its own included, in
    // split order.  Every access to the partials is an agent-scope (sc1)
    // store or load, performed at the level where all XCDs' L2s are
    // coherent, so no cache maintenance is needed: a block's stores have
    // reached that level when its s_waitcnt vmcnt(0) returns, which precedes
    // the block barrier and the device-scope ticket; the last block reads
    // only after its ticket has returned.  Release / acquire fences
    // (buffer_wbl2 / buffer_inv of a whole L2 per block) cost 12288 x 4096
    // at M = 128 22 us with 2 splits and 62 us with 5, for the same bits.
    const int tile = tm * tiles_n + tn - whole;  // among the split tiles
    float* Pb = P + (int64_t)tile * splits * (BM * RQ_BN);
    {
        float* mine = Pb + (int64_t)z * (BM * RQ_BN) + (wave * 64 + lane) * 4;
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4_t v = {acc[i][4 * g], acc[i][4 * g + 1], acc[i][4 * g + 2], acc[i][4 * g + 3]};
                rq_st16(mine + (i * 4 + g) * (RQ_NW * 64 * 4), v);
            }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        last_split = __hip_atomic_fetch_add(&cnt[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                     (uint32_t)(splits - 1);
    __syncthreads();
    if (!last_split) return;
    const float* Pl = Pb + (wave * 64 + lane) * 4;
#pragma unroll 1
    for (int i = 0; i < MT; ++i) {
        float v[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = 0.0f;
        // four splits' 16-B pieces in flight at a time, added in split order
        for (int s0 = 0; s0 < splits; s0 += 4) {
            f32x4_t r[4][4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int sj = s0 + j < splits ? s0 + j : splits - 1;
#pragma unroll
                for (int g = 0; g < 4; ++g) rq_ld16(r[j][g], Pl + (int64_t)sj * (BM * RQ_BN) + (i * 4 + g) * (RQ_NW * 64 * 4));
            }
            rq_wait_vm4(r);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (s0 + j < splits)
#pragma unroll
                    for (int e = 0; e < 16; ++e) v[e] += r[j][e >> 2][e & 3];
        }
        store_tile(i, v);
    }
    if (threadIdx.x == 0) __hip_atomic_store(&cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int QT, int BM, bool GU>
hipError_t rq_launch(const RqPlan& p, const uint8_t* wq, const void* x, void* y, bool yf32, int M, int K, int64_t nout,
                     int64_t up_off, float* ws, uint32_t* cnt, hipStream_t s) {
    const int64_t tiles = (int64_t)p.tiles_n * p.tiles_m;
    const dim3 grid((unsigned)(p.whole + (tiles - p.whole) * p.splits));
    const bf16_t* xb = static_cast<const bf16_t*>(x);
    if (yf32)
        hipLaunchKernelGGL((k_gemm_rq<QT, BM, GU, float>), grid, dim3(64 * RQ_NW), 0, s, wq, xb, static_cast<float*>(y), ws,
                           cnt, M, K, nout, up_off, p.tiles_n, p.whole, p.splits, p.kps);
    else
        hipLaunchKernelGGL((k_gemm_rq<QT, BM, GU, bf16_t>), grid, dim3(64 * RQ_NW), 0, s, wq, xb, static_cast<bf16_t*>(y), ws,
                           cnt, M, K, nout, up_off, p.tiles_n, p.whole, p.splits, p.kps);
    return hipGetLastError();
}

template <int QT, bool GU>
hipError_t rq_bm(const RqPlan& p, const uint8_t* wq, const void* x, void* y, bool yf32, int M, int K, int64_t nout,
                 int64_t up_off, float* ws, uint32_t* cnt, hipStream_t s) {
    if (p.bm == 128) return rq_launch<QT, 128, GU>(p, wq, x, y, yf32, M, K, nout, up_off, ws, cnt, s);
    return rq_launch<QT, 256, GU>(p, wq, x, y, yf32, M, K, nout, up_off, ws, cnt, s);
}

int rq_env(const char* name) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : 0;
}

}  // namespace

bool gemm_rq_supported(int qtype, int64_t M, int64_t N_rows, int64_t K, bool gu) {
    if (qtype != 12 && qtype != 13) return false;
    if (M < 1 || M >= (1 << 24) || N_rows < 1 || K < 256 || K % 256) return false;
    if (gu && N_rows % 8) return false;  // each wave's 16 up rows start on a row quad
    const uint64_t wbytes = (uint64_t)((N_rows + 3) / 4) * (uint64_t)(K / 256) * 576;
    return wbytes < (1ull << 32) && (uint64_t)M * (uint64_t)K * 2 < (1ull << 32);
}

// Block tile 128 rows of M up to M = 128, else 256, by 256 weight rows; one
// block per CU (160 / 152 KB of LDS).  Fewer tiles than CUs: every tile's K
// is split until the grid fills the CUs once, at least 4 K steps per split.
// More: whole rounds of tiles run unsplit and a last, partial round of at
// most half the CUs is split in two (12288 x 4096 at M = 2048: 384 tiles =
// 256 whole + 128 in halves, 96 K steps per CU instead of 128).
RqPlan plan_gemm_rq(int64_t M, int64_t N_rows, int64_t K, bool gu, int cus) {
    RqPlan p;
    if (cus < 1) cus = 256;
    int bm = rq_env("THQ_RQ_BM");
    if (bm != 128 && bm != 256) bm = M <= 128 ? 128 : 256;
    p.bm = bm;
    const int64_t nout = gu ? N_rows / 2 : N_rows;
    p.tiles_n = (int)((nout + (gu ? RQ_BN / 2 : RQ_BN) - 1) / (gu ? RQ_BN / 2 : RQ_BN));
    p.tiles_m = (int)((M + bm - 1) / bm);
    const int T = (int)(K / RQ_BK);
    const int64_t tiles = (int64_t)p.tiles_n * p.tiles_m;
    const int max_split = T / 4 > 0 ? T / 4 : 1;
    int splits = rq_env("THQ_RQ_SPLITS");
    int64_t whole;
    if (tiles < cus) {
        if (splits < 1) splits = (int)(cus / tiles);
        whole = 0;
    } else {
        const int64_t rest = tiles % cus;
        if (splits < 1) splits = rest > 0 && 2 * rest <= cus ? 2 : 1;
        whole = tiles - rest;
    }
    if (splits > max_split) splits = max_split;
    if (splits < 1) splits = 1;
    p.kps = (T + splits - 1) / splits;
    p.splits = (T + p.kps - 1) / p.kps;  // no empty split
    if (p.splits == 1) whole = tiles;
    p.whole = (int)whole;
    const int64_t split_tiles = tiles - whole;
    p.counters = p.splits > 1 ? split_tiles : 0;
    p.workspace_bytes = p.splits > 1 ? (size_t)split_tiles * (size_t)p.splits * (size_t)bm * RQ_BN * sizeof(float) : 0;
    return p;
}

hipError_t launch_gemm_rq(const RqPlan& p, bool affine, const uint8_t* wq, const void* x, void* y, bool yf32, bool gu,
                          int M, int64_t N_rows, int K, float* ws, uint32_t* cnt, hipStream_t s) {
    if (p.splits > 1 && (!ws || !cnt)) return hipErrorInvalidValue;
    const int64_t nout = gu ? N_rows / 2 : N_rows;
    const int64_t up_off = gu ? N_rows / 2 : 0;
    if (affine)
        return gu ? rq_bm<13, true>(p, wq, x, y, yf32, M, K, nout, up_off, ws, cnt, s)
                  : rq_bm<13, false>(p, wq, x, y, yf32, M, K, nout, up_off, ws, cnt, s);
    return gu ? rq_bm<12, true>(p, wq, x, y, yf32, M, K, nout, up_off, ws, cnt, s)
              : rq_bm<12, false>(p, wq, x, y, yf32, M, K, nout, up_off, ws, cnt, s);
}

}  // namespace thq
