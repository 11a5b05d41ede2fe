// k_gemv_mfma.hip — decode GEMV for 1 <= M <= 8 bf16 activation rows on the
// matrix cores, with exact (unrounded) dequantized weights.
//
// Role: the m = 1..8 projections of the reference (AffineQmvT / AffineQmpp,
// engine/src/quant_kernel.rs:2964-3140, 3188-3738, routed by rows in
// QLin::linear_ps, engine/src/qwen35.rs:398-617) over GGUF Q4_K / Q8_0
// weights.  HBM-bound: every weight byte is read once with 16-B loads.
//
// Why MFMA for a GEMV: with M rows of x, a VALU dot product costs ~M/2
// instructions per weight; here the products run on v_mfma_f32_32x32x16_bf16
// and the VALU only converts packed weights to bf16 (one v_perm per two Q4_K
// weights) and applies the per-32-weight scales, independent of M.
//
// Exactness.  Q4_K weight = d1*q - m1 per 32-weight sub-block.  The B operand
// holds bf16(128 + q) (exact: bytes [q, 0x43]), so the MFMA gives
// A = sum x*(128 + q) over a sub-block, and
//     sum x*w = d1*A - (128*d1 + m1) * S,   S = sum x over the sub-block,
// with S computed once per block while the activations are staged in LDS.
// Q8_0: B = bf16(q) (exact for |q| <= 128), sum = d*A.
//
// Tiling.  A block owns 32 weight rows (gate/up: 16 gate + 16 up rows of the
// same outputs) over a K range (all of K, or one of `splits` ranges when the
// tiles alone cannot fill the GPU; split partials are summed in a fixed order
// by k_split_reduce).  The block stages its activation rows x[0..M) of that
// range in LDS (with the 32-wide sums S), while the first weight chunks are
// already in flight; its (up to 8) waves then split the range into slices of
// whole 256-wide chunks, loading the chunk after next while computing.
// Units are 64 weights.  Lane l: weight row n = l % 32, half g = l / 32:
//   Q4_K  lane loads piece g (bytes 16g..16g+15) of the unit's 32 nibble
//         bytes; low nibbles of bytes 16g+0..7 / 16g+8..15 feed two MFMAs of
//         the first sub-block (k = k0 + 16g + 0..7 / 8..15), high nibbles the
//         second sub-block (k0 + 32 + ...).
//   Q8_0  lane loads bytes 16g..16g+15 of each of the unit's two blocks, same
//         k mapping (first block = k0..k0+31, second = k0+32..k0+63).
//   Q6_K  a unit is one 64-weight step of the QL / QH planes (thq_dev.hpp,
//         q6k_layout); each MFMA takes one whole 16-weight scale group G,
//         lane half g supplying its positions 8g..8g+7: QL bytes 8g..8g+7
//         (groups 0 / 2 in the low / high nibbles) and 16+8g.. (groups 1 / 3),
//         QH bytes 8g..8g+7 (group G in bits 2G).  B = bf16(128 + code), and
//         per group sum x*w = s*(A - 160*S16), s = d*sc, S16 = sum x over the
//         group; the block's K range is at most 4096 (256 group sums in LDS).
// The MFMA output lane holds column n and rows 8*(e/4) + 4*g + e%4: with
// M <= 8 only e = 0..3 (rows 4g + e) are live, with M <= 16 e = 0..7.  Each wave accumulates its
// slice in registers; the block sums the slices in LDS in wave order
// (deterministic) and applies the epilogue.
#include "thq_dev.hpp"
#include "thq_kernels.hpp"
#include "thq_wave.hpp"

#include <type_traits>

namespace thq {

namespace {

__device__ __forceinline__ f32x16_t mfma32x16(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// low nibbles of the bytes of a, b (already masked to 4 bits) -> bf16(128 + q) x 8
__device__ __forceinline__ bf16x8_t nib_bf16x8(uint32_t a, uint32_t b) {
    const uint32_t C = 0x43434343u;
    return as_bf16x8(make_uint4(__builtin_amdgcn_perm(C, a, 0x04010400u), __builtin_amdgcn_perm(C, a, 0x04030402u),
                                __builtin_amdgcn_perm(C, b, 0x04010400u), __builtin_amdgcn_perm(C, b, 0x04030402u)));
}
// int8 bytes of a, b -> bf16(q) x 8 (exact)
__device__ __forceinline__ bf16x8_t i8_bf16x8(uint32_t a, uint32_t b) {
    auto cv = [](uint32_t w, int i) { return (float)(int8_t)(w >> (8 * i)); };
    return as_bf16x8(make_uint4(pack_bf16x2(cv(a, 0), cv(a, 1)), pack_bf16x2(cv(a, 2), cv(a, 3)),
                                pack_bf16x2(cv(b, 0), cv(b, 1)), pack_bf16x2(cv(b, 2), cv(b, 3))));
}

constexpr int MAXW = 8;          // waves per block
constexpr int XS_ELEMS = 32768;  // staged activations (bf16) per block: M * Kb <= 32768
constexpr int KB_MAX = 8192;     // K range of one block
constexpr int XCH = 8;           // staged 16-B activation chunks per thread: M * cpw / 2 <= XCH
constexpr int MMAX = 16;         // activation rows (E = 8 live accumulator rows per lane)
// with M > 8, M * cpw <= 2 * XCH leaves one chunk per wave: Kb <= MAXW * 256
constexpr int KB_MAX_E8 = MAXW * 256;

// Packed weights and scales of one chunk (4 units = one Q4_K superblock) of a
// wave's K slice.
template <int QT>
struct Chunk {
    uint4 w[QT != 8 ? 4 : 8];
    uint32_t s[4];
    uint2 h[4];   // Q6_K QH bytes per unit
    uint32_t d;   // Q6_K f16 d
};

template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

// X is not __restrict__: its loads must stay ordered before the weight loads
// by the compiler barrier in the staging step.
// Grid: tiles x splits blocks; block (tile, split) owns the tile's 32 weight
// rows over K range [split*Kb, (split+1)*Kb), Kb = waves * cpw * 256.
// Four waves per SIMD for every weight type: two 8-wave blocks per CU (64 KB
// of LDS each).  Q8_0 with four live rows would then spill 28 B per lane, so
// Q8_0 runs 3..8 rows on the single-buffered eight-row instances instead.
template <int QT, int E, int NX, bool GU, bool SPLIT, typename YT>
__global__ __launch_bounds__(512, 4) void k_gemv_mfma(const uint8_t* __restrict__ Wq, const uint8_t* __restrict__ Wa,
                                                  const bf16_t* X, void* __restrict__ Yv, int M, int K,
                                                  int64_t nout, int64_t up_off, int64_t nrows, int cpw, int splits,
                                                  float* __restrict__ amv, uint32_t* __restrict__ ami, int64_t am_ld) {
    // staged activation rows (row stride Kb + 8: rows start 16 B apart in bank
    // order), sub-block sums S[sb][8] and the cross-wave reduction buffer
    __shared__ __attribute__((aligned(16))) bf16_t xs[XS_ELEMS + 8 * MMAX];
    // Q4_K / affine: 32-wide sums (Kb / 32 <= 256); Q6_K: 16-wide sums (Kb <= 4096);
    // E = 8 (M <= 16): Kb <= 2048, at most 128 sums of 16 rows
    constexpr int SR = E > 4 ? MMAX : 8;
    __shared__ __attribute__((aligned(16))) float Ss[QT == 8 ? 1 : (E > 4 ? KB_MAX_E8 / 16 : KB_MAX / 32)][SR];
    // the cross-wave reduction reuses the staging buffer once all waves are done with it
    float(*red)[SR][32] = reinterpret_cast<float(*)[SR][32]>(&xs[0]);
    static_assert(MAXW * SR * 32 * 4 <= XS_ELEMS * 2, "reduction buffer exceeds the staging buffer");
    static_assert(E == 1 || E == 2 || E == 4 || E == 8, "live accumulator rows");

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nw = blockDim.x >> 6;
    const int n = lane & 31, g = lane >> 5;
    const int tile = blockIdx.x / splits, split = blockIdx.x - tile * splits;
    const int Kb = nw * cpw * 256;
    const int kb0 = split * Kb;
    const int XR = Kb + 8;

    int64_t row;
    bool valid;
    if (GU) {
        const int64_t o = (int64_t)tile * 16 + (n & 15);
        valid = o < nout;
        row = o + (n >= 16 ? up_off : 0);
    } else {
        row = (int64_t)tile * 32 + n;
        valid = row < nout;
    }
    if (!valid) row = 0;  // in-bounds reads; its scales are zeroed below
    const int c0 = kb0 / 256 + wave * cpw;  // first 256-wide chunk of this wave

    const uint8_t* pw;
    const uint8_t* ps;
    const uint8_t* ph = nullptr;
    const uint16_t* pd = nullptr;
    if (QT == 14) {
        const Q6Layout L = q6k_layout(nrows, K);
        pw = Wq + row * (K >> 1) + 8 * g;
        ph = Wq + L.qh + row * (K >> 2) + 8 * g;
        ps = Wq + L.sc + row * (K >> 4);
        pd = reinterpret_cast<const uint16_t*>(Wq + L.d) + row * (K >> 8);
    } else if (QT != 8) {
        const int nsb = K >> 8;
        pw = Wq + q4k_piece(row, nsb, 0, g, 0);
        ps = Wq + q4k_hdword(row, nsb, 0, 0);
    } else {
        // Q8_0 tiles: block b of the row at pw + 1024 b, chunk c's 8 scales at ps + 512 c
        pw = Wq + q8t_q(row, K >> 5, 0, g);
        ps = Wa + q8t_d(row, K >> 5, 0) * 2;
    }
    auto load = [&](Chunk<QT>& C, int c) {
        if constexpr (QT == 14) {
            // scales and d first (in-order wait counters)
            const uint4 sv = *reinterpret_cast<const uint4*>(ps + (int64_t)c * 16);
            C.s[0] = sv.x; C.s[1] = sv.y; C.s[2] = sv.z; C.s[3] = sv.w;
            C.d = pd[c];
            // one base per chunk: the unit offsets fold into the loads' immediates
            const uint8_t* qlc = pw + (int64_t)c * 128;
            const uint8_t* qhc = ph + (int64_t)c * 64;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint2 lo = *reinterpret_cast<const uint2*>(qlc + u * 32);
                const uint2 hi = *reinterpret_cast<const uint2*>(qlc + u * 32 + 16);
                C.w[u] = make_uint4(lo.x, lo.y, hi.x, hi.y);
                C.h[u] = *reinterpret_cast<const uint2*>(qhc + u * 16);
            }
        } else if (QT != 8) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                C.w[u] = *reinterpret_cast<const uint4*>(pw + (int64_t)c * 64 + u * 16);
                C.s[u] = *reinterpret_cast<const uint32_t*>(ps + (int64_t)c * 64 + u * 16);
            }
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                C.w[2 * u] = *reinterpret_cast<const uint4*>(pw + (int64_t)c * 8192 + u * 2048);
                C.w[2 * u + 1] = *reinterpret_cast<const uint4*>(pw + (int64_t)c * 8192 + u * 2048 + 1024);
                C.s[u] = *reinterpret_cast<const uint32_t*>(ps + (int64_t)c * 512 + u * 4);
            }
        }
    };
    // ---- stage x[0..M)[kb0 .. kb0+Kb) and the 32-wide sums S (Q4_K).  The
    // activation loads are issued first, then the first two weight chunks, so
    // that the (in-order) wait before the LDS writes covers only the x loads
    // and the weight reads overlap the staging and the first chunk's math.
    const int cpr = Kb >> 3;  // 16-B chunks per row (a multiple of 4)
    const int total = M * cpr;  // <= NX * blockDim.x
    // straight-line loads (clamped indices, both chunks always loaded) keep the
    // compiler's wait counts exact
    uint4 xv[NX];
#pragma unroll
    for (int i = 0; i < NX; ++i) {
        int ch = threadIdx.x + i * blockDim.x;
        ch = ch < total ? ch : total - 1;
        const int m = ch / cpr, c = ch - m * cpr;
        xv[i] = *reinterpret_cast<const uint4*>(X + (int64_t)m * K + kb0 + 8 * c);
    }
    // keep the x loads ahead of the weight loads (IR and machine scheduling)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    Chunk<QT> B0, B1;
    load(B0, c0);
    if constexpr (E <= 4) load(B1, cpw > 1 ? c0 + 1 : c0);  // E = 8 plans give one chunk per wave
#pragma unroll
    for (int i = 0; i < NX; ++i) {
        const int ch = threadIdx.x + i * blockDim.x;
        if (ch < total) {
            const int m = ch / cpr, c = ch - m * cpr;
            const uint4 v = xv[i];
            *reinterpret_cast<uint4*>(&xs[m * XR + 8 * c]) = v;
            if (QT == 14) {
                // lanes 2j, 2j+1 hold the 2 chunks of one 16-wide group (pairs stay whole)
                const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
                bf16x2_t p[4];
                __builtin_memcpy(p, &v, 16);
                float t = __builtin_amdgcn_fdot2_f32_bf16(p[0], one, 0.0f, false);
                t = __builtin_amdgcn_fdot2_f32_bf16(p[1], one, t, false);
                t = __builtin_amdgcn_fdot2_f32_bf16(p[2], one, t, false);
                t = __builtin_amdgcn_fdot2_f32_bf16(p[3], one, t, false);
                t = dpp_add<0xB1>(t);  // quad_perm [1,0,3,2]
                if ((c & 1) == 0) Ss[c >> 1][m] = t;
            } else if (QT != 8) {
                // lanes 4j..4j+3 hold the 4 chunks of one sub-block (quads stay whole)
                const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
                bf16x2_t p[4];
                __builtin_memcpy(p, &v, 16);
                float t = __builtin_amdgcn_fdot2_f32_bf16(p[0], one, 0.0f, false);
                t = __builtin_amdgcn_fdot2_f32_bf16(p[1], one, t, false);
                t = __builtin_amdgcn_fdot2_f32_bf16(p[2], one, t, false);
                t = __builtin_amdgcn_fdot2_f32_bf16(p[3], one, t, false);
                t = dpp_add<0xB1>(t);  // quad_perm [1,0,3,2]
                t = dpp_add<0x4E>(t);  // quad_perm [2,3,0,1]
                if ((c & 3) == 0) Ss[c >> 2][m] = t;
            }
        }
    }
    __syncthreads();

    // 32x32 A operand row n (clamped to M-1)
    const bf16_t* xa = &xs[(n < M ? n : M - 1) * XR + (QT == 14 ? 8 : 16) * g];
    const f32x16_t z16 = {};
    float tot[E];
#pragma unroll
    for (int e = 0; e < E; ++e) tot[e] = 0.0f;

    // E = 8: eight live rows per lane; left free, the compiler issues every
    // unit's MFMAs first and spills their results.  Pinning tot after each
    // unit (and a scheduling barrier) keeps one unit's MFMAs in flight.
    auto pin_e8 = [](float(&t)[E]) {
        if constexpr (E > 4) {
#pragma unroll
            for (int e = 0; e < E; ++e) asm volatile("" : "+v"(t[e]));
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto compute = [&](const Chunk<QT>& C, int c) {
        if constexpr (QT == 14) {
            const float dd = valid ? f16_to_f32((uint16_t)C.d) : 0.0f;
            const uint32_t M4 = 0x0F0F0F0Fu;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int kl = (c * 4 + u) * 64 - kb0;  // offset inside the staged range
                const uint4 q = C.w[u];
                const uint2 h = C.h[u];
                uint32_t lo[4], hi[4];
                lo[0] = (q.x & M4) | ((h.x & 0x03030303u) << 4);
                hi[0] = (q.y & M4) | ((h.y & 0x03030303u) << 4);
                lo[1] = (q.z & M4) | ((h.x & 0x0C0C0C0Cu) << 2);
                hi[1] = (q.w & M4) | ((h.y & 0x0C0C0C0Cu) << 2);
                lo[2] = ((q.x >> 4) & M4) | (h.x & 0x30303030u);
                hi[2] = ((q.y >> 4) & M4) | (h.y & 0x30303030u);
                lo[3] = ((q.z >> 4) & M4) | ((h.x >> 2) & 0x30303030u);
                hi[3] = ((q.w >> 4) & M4) | ((h.y >> 2) & 0x30303030u);
#pragma unroll
                for (int G = 0; G < 4; ++G) {
                    const uint4 a = *reinterpret_cast<const uint4*>(xa + kl + 16 * G);
                    f32x4_t S[E > 4 ? 2 : 1];
#pragma unroll
                    for (int h = 0; h < (E > 4 ? 2 : 1); ++h)
                        S[h] = *reinterpret_cast<const f32x4_t*>(&Ss[(kl >> 4) + G][8 * h + 4 * g]);
                    const float sg = dd * (float)(int)(int8_t)(C.s[u] >> (8 * G));
                    const f32x16_t A = mfma32x16(as_bf16x8(a), nib_bf16x8(lo[G], hi[G]), z16);
#pragma unroll
                    for (int e = 0; e < E; ++e)
                        tot[e] = __builtin_fmaf(sg, __builtin_fmaf(-160.0f, S[e >> 2][e & 3], A[e]), tot[e]);
                    // the 16 MFMAs of a chunk are independent: left free, the compiler
                    // issues them all first and sinks their FMAs past the next chunk's
                    // loads, keeping every accumulator live; pinning tot here (and a
                    // scheduling barrier) keeps one group in flight at a time
#pragma unroll
                    for (int e = 0; e < E; ++e) asm volatile("" : "+v"(tot[e]));
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            return;
        }
        float d = 0.0f, dm = 0.0f;
        if (QT == 12) {
            d = f16_to_f32((uint16_t)__builtin_amdgcn_perm(C.s[1], C.s[0], 0x0c0c0703u));
            dm = f16_to_f32((uint16_t)__builtin_amdgcn_perm(C.s[3], C.s[2], 0x0c0c0703u));
            if (!valid) d = dm = 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int kl = (c * 4 + u) * 64 - kb0;  // offset inside the staged range
            const uint4 a0 = *reinterpret_cast<const uint4*>(xa + kl);
            const uint4 a1 = *reinterpret_cast<const uint4*>(xa + kl + 8);
            const uint4 a2 = *reinterpret_cast<const uint4*>(xa + kl + 32);
            const uint4 a3 = *reinterpret_cast<const uint4*>(xa + kl + 40);
            if (QT != 8) {
                f32x4_t S1[E > 4 ? 2 : 1], S2[E > 4 ? 2 : 1];
#pragma unroll
                for (int h = 0; h < (E > 4 ? 2 : 1); ++h) {
                    S1[h] = *reinterpret_cast<const f32x4_t*>(&Ss[kl >> 5][8 * h + 4 * g]);
                    S2[h] = *reinterpret_cast<const f32x4_t*>(&Ss[(kl >> 5) + 1][8 * h + 4 * g]);
                }
                const uint32_t h = C.s[u];
                float d1, d2, c1, c2;
                if constexpr (QT == 13) {  // affine group: w = scale * q + bias
                    const float sc = valid ? aff_scale(h) : 0.0f, bi = valid ? aff_bias(h) : 0.0f;
                    d1 = d2 = sc;
                    c1 = c2 = __builtin_fmaf(128.0f, sc, -bi);
                } else {
                    d1 = d * (float)(h & 63u);
                    d2 = d * (float)((h >> 12) & 63u);
                    c1 = __builtin_fmaf(128.0f, d1, dm * (float)((h >> 6) & 63u));
                    c2 = __builtin_fmaf(128.0f, d2, dm * (float)((h >> 18) & 63u));
                }
                const uint4 q = C.w[u];
                const uint32_t M4 = 0x0F0F0F0Fu;
                // one sub-block at a time keeps a single 16-register accumulator live
                f32x16_t A = mfma32x16(as_bf16x8(a0), nib_bf16x8(q.x & M4, q.y & M4), z16);
                A = mfma32x16(as_bf16x8(a1), nib_bf16x8(q.z & M4, q.w & M4), A);
#pragma unroll
                for (int e = 0; e < E; ++e)
                    tot[e] = __builtin_fmaf(-c1, S1[e >> 2][e & 3], __builtin_fmaf(d1, A[e], tot[e]));
                A = mfma32x16(as_bf16x8(a2), nib_bf16x8((q.x >> 4) & M4, (q.y >> 4) & M4), z16);
                A = mfma32x16(as_bf16x8(a3), nib_bf16x8((q.z >> 4) & M4, (q.w >> 4) & M4), A);
#pragma unroll
                for (int e = 0; e < E; ++e)
                    tot[e] = __builtin_fmaf(-c2, S2[e >> 2][e & 3], __builtin_fmaf(d2, A[e], tot[e]));
                pin_e8(tot);
            } else {
                float da = f16_to_f32((uint16_t)C.s[u]), db = f16_to_f32((uint16_t)(C.s[u] >> 16));
                if (!valid) da = db = 0.0f;
                const uint4 q0 = C.w[2 * u], q1 = C.w[2 * u + 1];
                f32x16_t A = mfma32x16(as_bf16x8(a0), i8_bf16x8(q0.x, q0.y), z16);
                A = mfma32x16(as_bf16x8(a1), i8_bf16x8(q0.z, q0.w), A);
#pragma unroll
                for (int e = 0; e < E; ++e) tot[e] = __builtin_fmaf(da, A[e], tot[e]);
                A = mfma32x16(as_bf16x8(a2), i8_bf16x8(q1.x, q1.y), z16);
                A = mfma32x16(as_bf16x8(a3), i8_bf16x8(q1.z, q1.w), A);
#pragma unroll
                for (int e = 0; e < E; ++e) tot[e] = __builtin_fmaf(db, A[e], tot[e]);
                pin_e8(tot);
            }
        }
    };

    // two chunk buffers; the chunk after next loads while a chunk computes
    if constexpr (E > 4) {
        compute(B0, c0);
    } else for (int c = 0; c < cpw; c += 2) {
        compute(B0, c0 + c);
        if (c + 2 < cpw) load(B0, c0 + c + 2);
        if (c + 1 >= cpw) break;
        compute(B1, c0 + c + 1);
        if (c + 3 < cpw) load(B1, c0 + c + 3);
    }

    // ---- block reduction over the waves' K slices, in wave order
    __syncthreads();  // every wave is done reading xs
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int m = 8 * (e >> 2) + 4 * g + (e & 3);
        if (m < M) red[wave][m][n] = tot[e];
    }
    __syncthreads();
    // outputs are strided over the block: a block may have fewer threads than 32*M
    if (SPLIT) {
        // f32 partial in natural weight-row order: P[split][m][row]
        for (int t = threadIdx.x; t < 32 * M; t += blockDim.x) {
            const int c = t & 31, m = t >> 5;
            float sum = 0.0f;
            for (int w = 0; w < nw; ++w) sum += red[w][m][c];
            int64_t r;
            bool ok;
            if (GU) {
                const int64_t o = (int64_t)tile * 16 + (c & 15);
                ok = o < nout;
                r = o + (c >= 16 ? up_off : 0);
            } else {
                r = (int64_t)tile * 32 + c;
                ok = r < nout;
            }
            if (ok) static_cast<float*>(Yv)[((int64_t)split * M + m) * nrows + r] = sum;
        }
    } else if (GU) {
        for (int t = threadIdx.x; t < 16 * M; t += blockDim.x) {
            const int c = t & 15, m = t >> 4;
            float gs = 0.0f, us = 0.0f;
            for (int w = 0; w < nw; ++w) {
                gs += red[w][m][c];
                us += red[w][m][c + 16];
            }
            const int64_t o = (int64_t)tile * 16 + c;
            if (o < nout) store_y<YT>(static_cast<YT*>(Yv) + (int64_t)m * nout + o, silu_mul(gs, us));
        }
    } else if (amv) {
        // fused argmax: the tile's 32 outputs per row (summed exactly as the
        // stored path sums them) reduce across their 32 lanes to (max, lowest
        // index) without a store; rows are whole half-waves
        for (int t0 = 0; t0 < 32 * M; t0 += blockDim.x) {
            const int t = t0 + threadIdx.x;
            const int c = t & 31, m = t >> 5;
            const int64_t o = (int64_t)tile * 32 + c;
            float v = -INFINITY;
            if (m < M) {
                float sum = 0.0f;
                for (int w = 0; w < nw; ++w) sum += red[w][m][c];
                if (o < nout) v = amax_key(sum);
            }
            uint32_t i = (uint32_t)o;
            amax_row32(v, i);
            if (m < M && c == 0) {
                amv[m * am_ld + tile] = v;
                ami[m * am_ld + tile] = i;
            }
        }
    } else {
        for (int t = threadIdx.x; t < 32 * M; t += blockDim.x) {
            const int c = t & 31, m = t >> 5;
            float sum = 0.0f;
            for (int w = 0; w < nw; ++w) sum += red[w][m][c];
            const int64_t o = (int64_t)tile * 32 + c;
            if (o < nout) store_y<YT>(static_cast<YT*>(Yv) + (int64_t)m * nout + o, sum);
        }
    }
}

int env_int(const char* name) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : 0;
}

template <int QT, int E, int NX, bool GU, typename YT>
hipError_t run(const GemvPlan& p, const WeightView& w, const bf16_t* x, void* y, int M, int64_t nout, int64_t up_off,
               float* ws, hipStream_t s, AmaxOut* am) {
    const int64_t tiles = GU ? (nout + 15) / 16 : (nout + 31) / 32;
    const dim3 grid((unsigned)(tiles * p.splits)), block(64 * p.waves);
    if (p.splits == 1) {
        float* amv = nullptr;
        uint32_t* ami = nullptr;
        int64_t ld = 0;
        if (am) {
            if (GU || tiles > am->ld) return hipErrorInvalidValue;
            amv = am->v;
            ami = am->i;
            ld = am->ld;
            am->nb = tiles;
        }
        hipLaunchKernelGGL((k_gemv_mfma<QT, E, NX, GU, false, YT>), grid, block, 0, s, w.q, w.aux, x, y, M,
                           (int)w.K, nout, up_off, w.N, p.cpw, 1, amv, ami, ld);
        return hipGetLastError();
    }
    if (am) return hipSuccess;  // split-K: no fused epilogue (am->nb stays 0)
    hipLaunchKernelGGL((k_gemv_mfma<QT, E, NX, GU, true, float>), grid, block, 0, s, w.q, w.aux, x, (void*)ws, M,
                       (int)w.K, nout, up_off, w.N, p.cpw, p.splits, (float*)nullptr, (uint32_t*)nullptr,
                       (int64_t)0);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_split_reduce(ws, y, std::is_same<YT, float>::value, GU, M, nout, up_off, w.N, p.splits, s);
}

}  // namespace

// The instance a plan runs: live accumulator rows per lane E (rows
// 8 * (e / 4) + 4g + e % 4 < M, e < E) and staged 16-B activation chunks per
// thread NX (M * cpw * 256 / 8 / (64 * waves) = M * cpw / 2, rounded up to
// 1, 2, 4, 8).  E = 8 (M = 9..16, and Q8_0 from 3 rows) needs one chunk per
// wave, (M + 1) / 2 <= 8 staged chunks per thread.  {0, 0}: no instance.
GemvInstance gemv_mfma_instance(int qtype, int M, const GemvPlan& p) {
    GemvInstance r;
    if (!p.waves || M < 1 || M > MMAX) return r;
    if (M <= 2 || (qtype != 8 && M <= 8)) {
        r.E = M == 1 ? 1 : (M == 2 ? 2 : 4);
        const int need = (M * p.cpw + 1) / 2;
        r.NX = need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : 8;
        return r;
    }
    if (p.cpw != 1 || p.waves * 256 > KB_MAX_E8) return r;
    r.E = 8;
    r.NX = 8;
    return r;
}

namespace {

template <int QT, bool GU, typename YT>
hipError_t run_e(const GemvPlan& p, const WeightView& w, const bf16_t* x, void* y, int M, int64_t nout,
                 int64_t up_off, float* ws, hipStream_t s, AmaxOut* am) {
    const GemvInstance in = gemv_mfma_instance(QT, M, p);
#define THQ_RUN(E_, NX_) run<QT, E_, NX_, GU, YT>(p, w, x, y, M, nout, up_off, ws, s, am)
    if (in.E == 8) return THQ_RUN(8, 8);
    if constexpr (QT != 8) {
        if (in.E == 4) {
            if (in.NX == 1) return THQ_RUN(4, 1);
            if (in.NX == 2) return THQ_RUN(4, 2);
            if (in.NX == 4) return THQ_RUN(4, 4);
            return THQ_RUN(4, 8);
        }
    }
    if (in.E == 2) {
        if (in.NX == 1) return THQ_RUN(2, 1);
        if (in.NX == 2) return THQ_RUN(2, 2);
        if (in.NX == 4) return THQ_RUN(2, 4);
        return THQ_RUN(2, 8);
    }
    if (in.E == 1) {
        if (in.NX == 1) return THQ_RUN(1, 1);
        if (in.NX == 2) return THQ_RUN(1, 2);
        if (in.NX == 4) return THQ_RUN(1, 4);
        return THQ_RUN(1, 8);
    }
#undef THQ_RUN
    return hipErrorInvalidValue;
}

}  // namespace

GemvPlan plan_gemv_mfma(int qtype, int64_t M, int64_t N_rows, int64_t K, bool gu) {
    GemvPlan p;
    if (M < 1 || M > MMAX || K < 256 || K % 256 || K > (1 << 20)) return p;
    if (qtype != 8 && qtype != 12 && qtype != 13 && qtype != 14) return p;
    const int64_t nout = gu ? N_rows / 2 : N_rows;
    const int64_t tiles = gu ? (nout + 15) / 16 : (nout + 31) / 32;
    const int chunks = (int)(K / 256);
    const int fs = env_int("THQ_GEMV_SPLITS"), fw = env_int("THQ_GEMV_WAVES");
    // the eight-row (E = 8) instances take one chunk per wave.  Q8_0 uses them
    // from 3 rows: its four-row instances spill 28 B per lane, the single-
    // buffered E = 8 ones none (12288 x 4096, M = 3 / 4 / 5 / 8: 20.7 / 20.9 /
    // 21.5 / 22.0 -> 19.4 / 19.6 / 19.9 / 19.6 us; at M = 2 the two-row
    // instance is faster, 17.0 against 19.6 us, and Q4_K keeps four rows)
    const bool one_chunk = M > 8 || (qtype == 8 && M > 2);
    // fewest K splits that fit the staged activations and give >= 256 blocks
    // (else the most splits, up to 16, that fit); waves: the most (<= 8) that
    // divide the block's chunks with M * (chunks per wave) <= 2 * XCH
    for (int s = 1; s <= chunks && s <= 16; ++s) {
        if (chunks % s || (fs && s != fs)) continue;
        const int64_t kb = K / s;
        if (kb > KB_MAX || M * kb > XS_ELEMS || (qtype == 14 && kb > 4096)) continue;
        const int cps = chunks / s;
        int w = 0;
        for (int c = MAXW; c >= 1; --c)
            if (cps % c == 0 && (!fw || c == fw) && M * (cps / c) <= 2 * XCH && !(one_chunk && cps / c != 1)) {
                w = c;
                break;
            }
        if (!w) continue;
        p.splits = s;
        p.waves = w;
        p.cpw = cps / w;
        p.workspace_bytes = s > 1 ? (size_t)s * (size_t)M * (size_t)N_rows * sizeof(float) : 0;
        if (fs || tiles * s >= 256) break;
    }
    return p;
}

GemvLimits gemv_mfma_limits() {
    GemvLimits l;
    l.xs_elems = XS_ELEMS;
    l.xs_pad_elems = 8 * MMAX;
    l.kb_max = KB_MAX;
    l.kb_max_e8 = KB_MAX_E8;
    l.mmax = MMAX;
    l.max_waves = MAXW;
    l.sums_rows_e4 = KB_MAX / 32;
    l.sums_rows_e8 = KB_MAX_E8 / 16;
    l.sums_cols_e4 = 8;
    l.sums_cols_e8 = MMAX;
    return l;
}

hipError_t launch_gemv_mfma(const GemvPlan& p, const WeightView& w, const void* x, void* y, bool yf32, bool gu, int M,
                            int64_t nout, int64_t up_off, float* ws, hipStream_t s, AmaxOut* am) {
    if (!p.waves) return hipErrorInvalidValue;
    const bf16_t* xb = static_cast<const bf16_t*>(x);
    if (w.qtype == 12) {
        if (gu) return yf32 ? run_e<12, true, float>(p, w, xb, y, M, nout, up_off, ws, s, am)
                            : run_e<12, true, bf16_t>(p, w, xb, y, M, nout, up_off, ws, s, am);
        return yf32 ? run_e<12, false, float>(p, w, xb, y, M, nout, up_off, ws, s, am)
                    : run_e<12, false, bf16_t>(p, w, xb, y, M, nout, up_off, ws, s, am);
    }
    if (w.qtype == 13) {
        if (gu) return yf32 ? run_e<13, true, float>(p, w, xb, y, M, nout, up_off, ws, s, am)
                            : run_e<13, true, bf16_t>(p, w, xb, y, M, nout, up_off, ws, s, am);
        return yf32 ? run_e<13, false, float>(p, w, xb, y, M, nout, up_off, ws, s, am)
                    : run_e<13, false, bf16_t>(p, w, xb, y, M, nout, up_off, ws, s, am);
    }
    if (w.qtype == 14) {
        if (gu) return yf32 ? run_e<14, true, float>(p, w, xb, y, M, nout, up_off, ws, s, am)
                            : run_e<14, true, bf16_t>(p, w, xb, y, M, nout, up_off, ws, s, am);
        return yf32 ? run_e<14, false, float>(p, w, xb, y, M, nout, up_off, ws, s, am)
                    : run_e<14, false, bf16_t>(p, w, xb, y, M, nout, up_off, ws, s, am);
    }
    if (gu) return yf32 ? run_e<8, true, float>(p, w, xb, y, M, nout, up_off, ws, s, am)
                        : run_e<8, true, bf16_t>(p, w, xb, y, M, nout, up_off, ws, s, am);
    return yf32 ? run_e<8, false, float>(p, w, xb, y, M, nout, up_off, ws, s, am)
                : run_e<8, false, bf16_t>(p, w, xb, y, M, nout, up_off, ws, s, am);
}

}  // namespace thq
