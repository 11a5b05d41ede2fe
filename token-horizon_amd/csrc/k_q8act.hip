// k_q8act.hip — THQ_MODE_Q8ACT: candle's default CPU matmul semantics on gfx950.
//
// [ext] candle-core 0.11 k_quants::matmul((m, k, n), lhs, rhs_t, dst) first
// quantizes every activation row to the weight's VecDotType
// (BlockQ8_0::from_float for Q8_0 weights, BlockQ8K::from_float for Q4_K
// weights), then computes each output as T::vec_dot(k, w_row, x_row_q): an
// integer dot per block, scaled in f32.  Here the quantizers are
// bit-identical to candle's, and the integer block dots are exact
// (v_dot4_i32_i8).  Only the f32 order in which the block terms are summed
// differs from candle's.
//
// Quantized activations on the device (split planes, internal):
//   xq [M][K] i8
//   Q8_0: xd [M][K/32] f32 = f32(f16(d)), the value vec_dot multiplies by
//   Q8_K: xd [M][K/256] f32 d, xb [M][K/32] i16 sums of 32 quants
//         (pairs of GGML's 16-wide bsums)
// thq_quantize_act writes GGML blocks instead (34-B Q8_0, 292-B Q8_K).
//
// The quantizers are compiled with -ffp-contract=off: every product and
// quotient rounds as written, like the Rust code they follow.
#include "thq_dev.hpp"
#include "thq_kernels.hpp"

namespace thq {
namespace {

// ------------------------------------------------------------------ helpers
__device__ __forceinline__ void load4(const float* p, float (&v)[4]) {
    const float4 t = *reinterpret_cast<const float4*>(p);
    v[0] = t.x;
    v[1] = t.y;
    v[2] = t.z;
    v[3] = t.w;
}
__device__ __forceinline__ void load4(const bf16_t* p, float (&v)[4]) {
    const uint2 t = *reinterpret_cast<const uint2*>(p);
    v[0] = bf16_to_f32(t.x & 0xFFFFu);
    v[1] = bf16_to_f32(t.x >> 16);
    v[2] = bf16_to_f32(t.y & 0xFFFFu);
    v[3] = bf16_to_f32(t.y >> 16);
}

// Rust `f as i8`: saturating, NaN -> 0; returned as the byte's bits
__device__ __forceinline__ uint32_t as_i8_bits(float v) {
    if (v != v) return 0u;
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    return (uint32_t)(uint8_t)(int8_t)v;
}

__device__ __forceinline__ uint16_t f16_bits(float f) {
    const _Float16 h = (_Float16)f;  // round to nearest even, like half::f16::from_f32
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

template <int P>
__device__ __forceinline__ uint32_t quad_lane(uint32_t v) {  // lane P of each quad, to all four
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, P | (P << 2) | (P << 4) | (P << 6), 0xF, 0xF, false);
}
__device__ __forceinline__ int pair_sum(int v) {  // lanes 2i, 2i+1
    return v + __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
}
// DPP moves within a row of 16 lanes (no LDS traffic, unlike __shfl_xor's
// ds_bpermute): quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E, row_half_mirror
// (lane i <-> 7 - i of each 8) = 0x141, row_mirror (i <-> 15 - i) = 0x140
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}

__device__ __forceinline__ int quad_sum(int v) {
    v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    return v + __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
}

// Transposed wave reduction of N per-lane values (N a power of two <= 64):
// each step with a value count above one hands half of them to the partner
// lane, so N values cost about N shuffles.  Afterwards a[0] of lane L is the
// wave total of value tred_slot<N>(L).
template <int N, int OFF>
struct TRed {
    static __device__ __forceinline__ void run(float* a, int lane) {
        if constexpr (OFF == 0) {
            return;
        } else if constexpr (N > 1) {
            const bool up = lane & OFF;
#pragma unroll
            for (int i = 0; i < N / 2; ++i) {
                const float keep = up ? a[i + N / 2] : a[i];
                const float give = up ? a[i] : a[i + N / 2];
                a[i] = keep + __shfl_xor(give, OFF, 64);
            }
            TRed<N / 2, OFF / 2>::run(a, lane);
        } else {
            a[0] += __shfl_xor(a[0], OFF, 64);
            TRed<1, OFF / 2>::run(a, lane);
        }
    }
};

template <int N>
__device__ __forceinline__ int tred_slot(int lane) {
    int s = 0, n = N;
    for (int off = 32; off >= 1 && n > 1; off >>= 1, n >>= 1)
        if (lane & off) s += n / 2;
    return s;
}

// ------------------------------------------------------------------ activation quantizers
// Q8_0 ([ext] BlockQ8_0::from_float): 8 lanes per 32-wide block, 4 values
// per lane.  amax = max |x| from 0 (NaN never wins), d = amax / 127,
// id = d != 0 ? 1 / d : 0, q = round(x * id) as i8, stored d = f16(d).
template <typename XT, bool GGUF>
__global__ __launch_bounds__(256) void k_quant_act_q8_0(const XT* __restrict__ x, int64_t nq, int8_t* __restrict__ xq,
                                                        float* __restrict__ xd, uint8_t* __restrict__ blk) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool live = t < nq;  // nq is a multiple of 8: a block's lanes are all live or all not
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (live) load4(x + 4 * t, v);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) amax = fmaxf(amax, fabsf(v[i]));
    // the 8 lanes of the block: the two quads, then the half-row mirror
    amax = fmaxf(amax, dpp_f<0xB1>(amax));
    amax = fmaxf(amax, dpp_f<0x4E>(amax));
    amax = fmaxf(amax, dpp_f<0x141>(amax));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint32_t q = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) q |= as_i8_bits(roundf(v[i] * id)) << (8 * i);
    if (!live) return;
    const int64_t b = t >> 3;
    const int j = (int)(t & 7);
    const uint16_t dh = f16_bits(d);
    if constexpr (GGUF) {
        uint16_t* p = reinterpret_cast<uint16_t*>(blk + b * 34);  // 2-B aligned blocks
        if (j == 0) p[0] = dh;
        p[1 + 2 * j] = (uint16_t)(q & 0xFFFFu);
        p[2 + 2 * j] = (uint16_t)(q >> 16);
    } else {
        reinterpret_cast<uint32_t*>(xq)[t] = q;
        if (j == 0) xd[b] = f16_to_f32(dh);
    }
}

// Q8_K ([ext] BlockQ8K::from_float): one wave per 256-wide block, 4 values
// per lane.  max = the signed element of largest magnitude, the first one
// on equal magnitudes (NaN never wins); amax == 0 gives d = 0 and zero
// quants; else iscale = -128 / max, q = min(round(iscale * x), 127) as i8,
// d = 1 / iscale, bsums = sums of 16 quants.
struct Q8KLane {
    uint32_t q;  // the lane's four quants (bytes)
    float d;     // the block's d
    int s16;     // sum of the 16 quants of lanes 4j .. 4j+3 (every lane of the quad)
    int s32;     // sum of the 32 quants of lanes 8j .. 8j+7 (every lane of the octet)
};

// one wave quantizes one 256-wide block, lane l holding values 4l .. 4l+3;
// all 64 lanes active (the cross-lane steps read every lane)
__device__ __forceinline__ Q8KLane q8k_wave(const float (&v)[4], int lane) {
    float key = -1.0f, val = 0.0f;
    int idx = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = fabsf(v[i]);
        if (a > key) {
            key = a;
            idx = 4 * lane + i;
            val = v[i];
        }
    }
    // (largest magnitude, then lowest index) is a selection of one element,
    // so any combine order gives the same one: DPP within each row of 16
    // lanes (quads, half rows, rows), then the four rows' winners read out
    auto comb = [](float& ck, int& ci, float& cv, float ok, int oi, float ov) {
        if (ok > ck || (ok == ck && oi < ci)) {
            ck = ok;
            ci = oi;
            cv = ov;
        }
    };
    comb(key, idx, val, dpp_f<0xB1>(key), dpp_i<0xB1>(idx), dpp_f<0xB1>(val));
    comb(key, idx, val, dpp_f<0x4E>(key), dpp_i<0x4E>(idx), dpp_f<0x4E>(val));
    comb(key, idx, val, dpp_f<0x141>(key), dpp_i<0x141>(idx), dpp_f<0x141>(val));
    comb(key, idx, val, dpp_f<0x140>(key), dpp_i<0x140>(idx), dpp_f<0x140>(val));
    {
        float bk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(key), 0));
        int bi = __builtin_amdgcn_readlane(idx, 0);
        float bv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(val), 0));
#pragma unroll
        for (int r = 16; r < 64; r += 16)
            comb(bk, bi, bv, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(key), r)),
                 __builtin_amdgcn_readlane(idx, r), __int_as_float(__builtin_amdgcn_readlane(__float_as_int(val), r)));
        key = bk;
        idx = bi;
        val = bv;
    }
    Q8KLane r;
    r.q = 0;
    r.d = 0.0f;
    if (key > 0.0f) {
        const float iscale = -128.0f / val;
#pragma unroll
        for (int i = 0; i < 4; ++i) r.q |= as_i8_bits(fminf(roundf(iscale * v[i]), 127.0f)) << (8 * i);
        r.d = 1.0f / iscale;
    }
    int s = (int)(int8_t)(r.q & 0xFFu) + (int)(int8_t)((r.q >> 8) & 0xFFu) + (int)(int8_t)((r.q >> 16) & 0xFFu) +
            (int)(int8_t)(r.q >> 24);
    r.s16 = quad_sum(s);  // 16 quants: lanes 4j .. 4j+3
    r.s32 = r.s16 + dpp_i<0x141>(r.s16);  // the other quad of the 8
    return r;
}

template <typename XT, bool GGUF>
__global__ __launch_bounds__(256) void k_quant_act_q8k(const XT* __restrict__ x, int64_t nblk, int8_t* __restrict__ xq,
                                                       float* __restrict__ xd, int16_t* __restrict__ xb,
                                                       uint8_t* __restrict__ blk) {
    const int lane = threadIdx.x & 63;
    const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nblk) return;  // the whole wave
    float v[4];
    load4(x + b * 256 + 4 * lane, v);
    const Q8KLane r = q8k_wave(v, lane);
    const uint32_t q = r.q;
    const float d = r.d;
    const int s = r.s16, s32 = r.s32;
    if constexpr (GGUF) {
        uint8_t* p = blk + b * 292;  // 4-B aligned blocks
        if (lane == 0) *reinterpret_cast<float*>(p) = d;
        reinterpret_cast<uint32_t*>(p + 4)[lane] = q;
        if ((lane & 3) == 0) reinterpret_cast<int16_t*>(p + 260)[lane >> 2] = (int16_t)s;
    } else {
        reinterpret_cast<uint32_t*>(xq + b * 256)[lane] = q;
        if (lane == 0) xd[b] = d;
        if ((lane & 7) == 0) xb[b * 8 + (lane >> 3)] = (int16_t)s32;
    }
}

// ------------------------------------------------------------------ dot kernels
// A wave owns four outputs (gate/up: four gate rows and the four matching up
// rows) and walks K; a block of four waves shares MT activation rows staged
// in LDS.  Lanes accumulate f32 block terms; the NR x MT totals are reduced
// across the wave at the end with the transposed reduction.
template <bool GU>
__device__ __forceinline__ void wave_rows(int64_t (&rows)[GU ? 8 : 4], int64_t o0, int64_t nout, int64_t up_off) {
#pragma unroll
    for (int r = 0; r < (GU ? 8 : 4); ++r) {
        int64_t o = o0 + (r & 3);
        if (o >= nout) o = nout - 1;  // loads stay in bounds; the store is skipped
        rows[r] = (GU && r >= 4) ? o + up_off : o;
    }
}

// y[i] = v with a device-scope (agent) relaxed atomic store: written through
// to the device's coherence point, so another XCD can read it back with
// device-scope loads and no cache write-back or invalidation is needed
template <typename YT>
__device__ __forceinline__ void store_y_device(YT* p, float v) {
    if constexpr (sizeof(YT) == 4) {
        __hip_atomic_store(reinterpret_cast<float*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        __hip_atomic_store(reinterpret_cast<uint16_t*>(p), (uint16_t)f32_to_bf16(v), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int MT, bool GU, typename YT, bool COH = false>
__device__ __forceinline__ void q8act_store(float (&acc)[(GU ? 8 : 4) * MT], int lane, YT* __restrict__ y, int64_t o0,
                                            int64_t nout, int m0, int mrows, int64_t ldy) {
    constexpr int NV = (GU ? 8 : 4) * MT;
    constexpr int SPAN = 64 / NV;
    TRed<NV, 32>::run(acc, lane);
    const float tot = acc[0];
    const int slot = tred_slot<NV>(lane);
    const int r = slot / MT, m = slot - (slot / MT) * MT;
    if constexpr (GU) {
        const float u = __shfl_xor(tot, 32, 64);  // up slot = gate slot + NV/2
        if ((lane & (SPAN - 1)) || (lane & 32)) return;
        if (m < mrows && o0 + r < nout) {
            if constexpr (COH)
                store_y_device<YT>(y + (int64_t)(m0 + m) * ldy + o0 + r, silu_mul(tot, u));
            else
                store_y<YT>(y + (int64_t)(m0 + m) * ldy + o0 + r, silu_mul(tot, u));
        }
    } else {
        if (lane & (SPAN - 1)) return;
        if (m < mrows && o0 + r < nout) store_y<YT>(y + (int64_t)(m0 + m) * ldy + o0 + r, tot);
    }
}

// Q4_K weights x Q8_K activations ([ext] BlockQ4K::vec_dot).  Lane 4s'+p of
// a 4096-wide chunk takes part p (sub-blocks 2p, 2p+1) of superblock s: the
// two 16-B nibble pieces of each row and the row's header dword p.  Per
// superblock and row the quad forms the exact integers
//   aux = sum_j sc_j * (q4 . q8)_j,   mins = sum_j m_j * bsum32_j
// and adds (d_w * d_x) * aux - (dmin_w * d_x) * mins.
// LDS: x [MT][K/16] 16-B pieces (piece 4u + t of lane unit u at slot
// 4u + ((t + u/4) & 3), so a lane's four reads hit distinct banks), the
// 32-sum pairs [MT][K/64] u32 and d [MT][K/256] f32.
//
// EMIT (gate/up, nout a multiple of 256): the producer also writes the
// next projection's operand, the Q8_K planes of its own output y
// (xq [M][nout] i8, xd [M][nout/256] f32, xb [M][nout/32] i16, as
// thq_q8act_prepare writes them for x = y).  A block covers 16 outputs, so
// 16 blocks share one 256-wide Q8_K block of each row.  Each block stores
// its outputs with device-scope stores (written through to the coherence
// point shared by all XCDs), waits for them to complete, then takes a ticket
// on the counter of its (row tile, 256-wide segment); the 16th block to
// arrive reads the segment of y back with device-scope loads and quantizes
// it, one wave per row, then resets the counter to 0 for the next launch.
// No block waits on another, and no cache is written back or invalidated
// (a device-scope fence per block, which writes back the whole L2, made the
// layer 2.4x slower).
template <int MT, bool GU, typename YT, bool EMIT = false>
__global__ __launch_bounds__(256) void k_q8act_q4k(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                   const float* __restrict__ xd, const int16_t* __restrict__ xb,
                                                   YT* __restrict__ y, int M, int64_t nout, int K, int64_t up_off,
                                                   int64_t ldy, uint32_t* __restrict__ cnt, int8_t* __restrict__ oq,
                                                   float* __restrict__ od, int16_t* __restrict__ ob) {
    constexpr int NR = GU ? 8 : 4;
    extern __shared__ uint4 lds4[];
    const int nsb = K >> 8, nu = K >> 6, npc = K >> 4;
    const int m0 = blockIdx.y * MT;
    const int mrows = M - m0 < MT ? M - m0 : MT;
    uint4* xs = lds4;
    uint32_t* bsl = reinterpret_cast<uint32_t*>(lds4 + MT * npc);
    float* dxl = reinterpret_cast<float*>(bsl + MT * nu);
    for (int i = threadIdx.x; i < MT * npc; i += 256) {
        const int m = i / npc, P = i - m * npc;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (m < mrows) v = reinterpret_cast<const uint4*>(xq + (int64_t)(m0 + m) * K)[P];
        const int u = P >> 2, t = P & 3;
        xs[m * npc + 4 * u + ((t + (u >> 2)) & 3)] = v;
    }
    for (int i = threadIdx.x; i < MT * nu; i += 256) {
        const int m = i / nu, u = i - m * nu;
        bsl[i] = m < mrows ? reinterpret_cast<const uint32_t*>(xb + (int64_t)(m0 + m) * (K >> 5))[u] : 0u;
    }
    for (int i = threadIdx.x; i < MT * nsb; i += 256) {
        const int m = i / nsb, s = i - m * nsb;
        dxl[i] = m < mrows ? xd[(int64_t)(m0 + m) * nsb + s] : 0.0f;
    }
    __syncthreads();

    const int lane = threadIdx.x & 63, p = lane & 3;
    const int64_t o0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 4;
    int64_t rows[NR];
    wave_rows<GU>(rows, o0, nout, up_off);
    float acc[NR * MT];
#pragma unroll
    for (int i = 0; i < NR * MT; ++i) acc[i] = 0.0f;
    const int nch = (nsb + 15) >> 4;
    for (int c = 0; c < nch; ++c) {
        const int s = 16 * c + (lane >> 2);
        const bool live = s < nsb;
        const int sl = live ? s : nsb - 1;
        uint4 w0[NR], w1[NR];
        uint32_t hw[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            w0[r] = *reinterpret_cast<const uint4*>(W + q4k_piece(rows[r], nsb, sl, 0, p));
            w1[r] = *reinterpret_cast<const uint4*>(W + q4k_piece(rows[r], nsb, sl, 1, p));
            hw[r] = *reinterpret_cast<const uint32_t*>(W + q4k_hdword(rows[r], nsb, sl, p));
        }
        float dw[NR], dmw[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const uint32_t t0 = quad_lane<0>(hw[r]), t1 = quad_lane<1>(hw[r]);
            const uint32_t t2 = quad_lane<2>(hw[r]), t3 = quad_lane<3>(hw[r]);
            dw[r] = f16_to_f32((uint16_t)__builtin_amdgcn_perm(t1, t0, 0x0c0c0703u));
            dmw[r] = f16_to_f32((uint16_t)__builtin_amdgcn_perm(t3, t2, 0x0c0c0703u));
        }
        const int u = 4 * sl + p;  // lane unit in the row
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            uint4 xv[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) xv[t] = xs[m * npc + 4 * u + ((t + (u >> 2)) & 3)];
            const uint32_t bs = bsl[m * nu + u];
            const int bs0 = (int)(int16_t)(bs & 0xFFFFu), bs1 = (int)(int16_t)(bs >> 16);
            const float dx = dxl[m * nsb + sl];
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const uint32_t M4 = 0x0F0F0F0Fu;
                int dlo = sdot4(w0[r].x & M4, xv[0].x, 0);
                dlo = sdot4(w0[r].y & M4, xv[0].y, dlo);
                dlo = sdot4(w0[r].z & M4, xv[0].z, dlo);
                dlo = sdot4(w0[r].w & M4, xv[0].w, dlo);
                dlo = sdot4(w1[r].x & M4, xv[1].x, dlo);
                dlo = sdot4(w1[r].y & M4, xv[1].y, dlo);
                dlo = sdot4(w1[r].z & M4, xv[1].z, dlo);
                dlo = sdot4(w1[r].w & M4, xv[1].w, dlo);
                int dhi = sdot4((w0[r].x >> 4) & M4, xv[2].x, 0);
                dhi = sdot4((w0[r].y >> 4) & M4, xv[2].y, dhi);
                dhi = sdot4((w0[r].z >> 4) & M4, xv[2].z, dhi);
                dhi = sdot4((w0[r].w >> 4) & M4, xv[2].w, dhi);
                dhi = sdot4((w1[r].x >> 4) & M4, xv[3].x, dhi);
                dhi = sdot4((w1[r].y >> 4) & M4, xv[3].y, dhi);
                dhi = sdot4((w1[r].z >> 4) & M4, xv[3].z, dhi);
                dhi = sdot4((w1[r].w >> 4) & M4, xv[3].w, dhi);
                const uint32_t h = hw[r];
                const int sc0 = (int)(h & 63u), mn0 = (int)((h >> 6) & 63u);
                const int sc1 = (int)((h >> 12) & 63u), mn1 = (int)((h >> 18) & 63u);
                const int aux = quad_sum(sc0 * dlo + sc1 * dhi);
                const int mins = quad_sum(mn0 * bs0 + mn1 * bs1);
                const float dd = dw[r] * dx, dm = dmw[r] * dx;
                const float a = __builtin_fmaf(-dm, (float)mins, __builtin_fmaf(dd, (float)aux, acc[r * MT + m]));
                acc[r * MT + m] = live ? a : acc[r * MT + m];
            }
        }
    }
#pragma unroll
    for (int i = 0; i < NR * MT; ++i) acc[i] = p == 0 ? acc[i] : 0.0f;  // one lane per quad
    q8act_store<MT, GU, YT, EMIT>(acc, lane, y, o0, nout, m0, mrows, ldy);
    if constexpr (EMIT) {
        // the outputs went out as device-scope (sc1) stores, published before
        // the ticket (ticket_publish, thq_dev.hpp) and read back with
        // device-scope loads after it
        __shared__ int last;
        const int64_t seg = blockIdx.x >> 4;  // 256-wide segment of the outputs
        uint32_t* c = cnt + (int64_t)blockIdx.y * (nout >> 8) + seg;
        ticket_publish();
        __syncthreads();
        if (threadIdx.x == 0) last = ticket_draw(c) == 15u;
        __syncthreads();
        if (last) {
            const int wave = threadIdx.x >> 6;
            const int nsb = (int)(nout >> 8);
            for (int m = wave; m < mrows; m += 4) {
                const int64_t row = m0 + m;
                float v[4];
                const YT* src = y + row * ldy + seg * 256 + 4 * lane;
                if constexpr (sizeof(YT) == 4) {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        v[i] = __hip_atomic_load(reinterpret_cast<const float*>(src) + i, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
                } else {
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const uint32_t t = __hip_atomic_load(reinterpret_cast<const uint32_t*>(src) + i,
                                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        v[2 * i] = bf16_to_f32(t & 0xFFFFu);
                        v[2 * i + 1] = bf16_to_f32(t >> 16);
                    }
                }
                const Q8KLane r = q8k_wave(v, lane);
                reinterpret_cast<uint32_t*>(oq + row * nout + seg * 256)[lane] = r.q;
                if (lane == 0) od[row * nsb + seg] = r.d;
                if ((lane & 7) == 0) ob[row * (nout >> 5) + seg * 8 + (lane >> 3)] = (int16_t)r.s32;
            }
            if (threadIdx.x == 0) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // for the next launch
        }
    }
}

// Q8_0 weights x Q8_0 activations ([ext] BlockQ8_0::vec_dot: per block
// (sum q_w q_x) * (d_w * d_x)) on the tile planes (thq_dev.hpp, q8t_q /
// q8t_d).  A wave takes one 32-row tile over a range of 256-wide chunks (a
// block's four waves: TPB = 4 / KS tiles x KS ranges of K).  Per block of K,
// one v_mfma_i32_32x32x32_i8 forms every (activation row, weight row) block
// integer exactly: B = the tile's 1-KB block as loaded (lane (n, g): row n's
// 16 bytes of half g), A = the x rows' 16 bytes of the same half (LDS; lanes
// past the call's rows hold zero).  Lane (n, g) then adds
// (d_w * d_x) * integer for weight row n and activation rows 4g .. 4g + 3 in
// block order; the K ranges are summed in order in LDS at the end.
// LDS: x [MT][K] i8, d_x [K/32][8] f32.
typedef int q8i32x4 __attribute__((ext_vector_type(4)));
typedef int q8i32x16 __attribute__((ext_vector_type(16)));
template <int MT, int KS, bool GU, typename YT>
__global__ __launch_bounds__(256) void k_q8act_q8_0(const int8_t* __restrict__ Q, const uint16_t* __restrict__ D,
                                                    const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                    YT* __restrict__ y, int M, int64_t nout, int K, int64_t up_off,
                                                    int64_t ldy) {
    static_assert(MT >= 1 && MT <= 8, "activation rows 4g .. 4g + 3 of the two lane halves");
    constexpr int TPB = 4 / KS;
    constexpr int R = GU ? 2 : 1;
    extern __shared__ uint4 lds4[];
    __shared__ float red[KS > 1 ? KS - 1 : 1][TPB][64][4 * R];
    const int nb = K >> 5, npc = K >> 4;
    const int m0 = blockIdx.y * MT;
    const int mrows = M - m0 < MT ? M - m0 : MT;
    uint4* xs = lds4;
    float* dxl = reinterpret_cast<float*>(lds4 + MT * npc);
    for (int i = threadIdx.x; i < MT * npc; i += 256) {
        const int m = i / npc, P = i - m * npc;
        xs[i] = m < mrows ? reinterpret_cast<const uint4*>(xq + (int64_t)(m0 + m) * K)[P] : make_uint4(0u, 0u, 0u, 0u);
    }
    for (int i = threadIdx.x; i < nb * 8; i += 256) {
        const int bb = i >> 3, m = i & 7;
        dxl[i] = m < mrows ? xd[(int64_t)(m0 + m) * nb + bb] : 0.0f;
    }
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 31, g = lane >> 5;
    const int ti = wave % TPB, ks = wave / TPB;
    const int64_t o = ((int64_t)blockIdx.x * TPB + ti) * 32 + n;
    const bool live = o < nout;
    int64_t rows[R];
    rows[0] = GU ? (live ? o : 0) : o;  // padding rows of the last tile hold zero weights
    if constexpr (GU) rows[R - 1] = live ? o + up_off : 0;
    const int8_t* pq[R];
    const uint16_t* pd[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        pq[r] = Q + q8t_q(rows[r], nb, 0, g);
        pd[r] = D + q8t_d(rows[r], nb, 0);
    }
    const bool arow = n < mrows;  // A operand row n = activation row m0 + n
    const int nch = (nb + 7) >> 3;
    const int cpk = (nch + KS - 1) / KS;
    const int c0 = ks * cpk, c1 = c0 + cpk < nch ? c0 + cpk : nch;
    float acc[R][4];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[r][e] = 0.0f;
    const q8i32x16 z16 = {};
    q8i32x4 av = {0, 0, 0, 0};
    for (int c = c0; c < c1; ++c) {
        const int nbc = nb - 8 * c < 8 ? nb - 8 * c : 8;
        uint4 dv[R];
        uint4 q[R][8];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            dv[r] = *reinterpret_cast<const uint4*>(pd[r] + (int64_t)c * 256);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                q[r][j] = j < nbc ? *reinterpret_cast<const uint4*>(pq[r] + ((int64_t)c * 8 + j) * 1024)
                                  : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (j < nbc) {
                const int bb = 8 * c + j;
                if (arow) {
                    const uint4 xv = xs[n * npc + 2 * bb + g];
                    av = q8i32x4{(int)xv.x, (int)xv.y, (int)xv.z, (int)xv.w};
                }
                const f32x4_t dx = *reinterpret_cast<const f32x4_t*>(&dxl[bb * 8 + 4 * g]);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint32_t w = j < 2 ? dv[r].x : (j < 4 ? dv[r].y : (j < 6 ? dv[r].z : dv[r].w));
                    const float dw = f16_to_f32((uint16_t)((j & 1) ? (w >> 16) : w));
                    const q8i32x4 bv = {(int)q[r][j].x, (int)q[r][j].y, (int)q[r][j].z, (int)q[r][j].w};
                    const q8i32x16 C = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, z16, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[r][e] = __builtin_fmaf(dw * dx[e], (float)C[e], acc[r][e]);
                }
            }
        }
    }
    if constexpr (KS > 1) {
        if (ks > 0) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int e = 0; e < 4; ++e) red[ks - 1][ti][lane][4 * r + e] = acc[r][e];
        }
        __syncthreads();
        if (ks == 0) {
#pragma unroll
            for (int k = 0; k < KS - 1; ++k)
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[r][e] += red[k][ti][lane][4 * r + e];
        }
    }
    if (ks == 0 && live) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int m = 4 * g + e;
            if (m < mrows)
                store_y<YT>(y + (int64_t)(m0 + m) * ldy + o, GU ? silu_mul(acc[0][e], acc[R - 1][e]) : acc[0][e]);
        }
    }
}

// ------------------------------------------------------------------ host side
constexpr size_t kLdsCap = 64 * 1024;

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

size_t lds_bytes(int qtype, int mt, int K) {
    const size_t x = (size_t)mt * K;
    return qtype == 12 ? x + (size_t)mt * (K / 64) * 4 + (size_t)mt * (K / 256) * 4 : x + (size_t)(K / 32) * 8 * 4;
}

int pick_mt(int qtype, int64_t M, int K) {
    int mt = 8;
    while (mt > 1 && mt / 2 >= M) mt /= 2;
    while (mt > 1 && lds_bytes(qtype, mt, K) > kLdsCap) mt /= 2;
    return mt;
}

struct ActPlanes {
    int8_t* xq;
    float* xd;
    int16_t* xb;
};

ActPlanes act_planes(int qtype, void* ws, int64_t M, int64_t K) {
    char* p = static_cast<char*>(ws);
    ActPlanes a;
    a.xq = reinterpret_cast<int8_t*>(p);
    p += align256((size_t)M * K);
    a.xd = reinterpret_cast<float*>(p);
    p += align256((size_t)M * (K / (qtype == 12 ? 256 : 32)) * 4);
    a.xb = reinterpret_cast<int16_t*>(p);
    return a;
}

// the planes of rows r0.. of a plane set with rows of K activations
ActPlanes act_rows(const ActPlanes& a, int qtype, int64_t K, int64_t r0) {
    ActPlanes r;
    r.xq = a.xq + r0 * K;
    r.xd = a.xd + r0 * (K / (qtype == 12 ? 256 : 32));
    r.xb = a.xb + r0 * (K / 32);
    return r;
}

// Row tiles go in grid.y, at most 65535 per launch: larger M runs as
// several launches over row chunks (stream-ordered).
constexpr int64_t kMaxGridY = 65535;

template <typename XT>
hipError_t quant_act_t(int qtype, const XT* x, int64_t M, int64_t K, const ActPlanes* pl, uint8_t* blocks,
                       hipStream_t s) {
    if (qtype == 8) {
        const int64_t nq = M * K / 4;
        const dim3 grid((unsigned)((nq + 255) / 256));
        if (blocks)
            hipLaunchKernelGGL((k_quant_act_q8_0<XT, true>), grid, dim3(256), 0, s, x, nq, nullptr, nullptr, blocks);
        else
            hipLaunchKernelGGL((k_quant_act_q8_0<XT, false>), grid, dim3(256), 0, s, x, nq, pl->xq, pl->xd, nullptr);
    } else {
        const int64_t nblk = M * K / 256;
        const dim3 grid((unsigned)((nblk + 3) / 4));
        if (blocks)
            hipLaunchKernelGGL((k_quant_act_q8k<XT, true>), grid, dim3(256), 0, s, x, nblk, nullptr, nullptr, nullptr,
                               blocks);
        else
            hipLaunchKernelGGL((k_quant_act_q8k<XT, false>), grid, dim3(256), 0, s, x, nblk, pl->xq, pl->xd, pl->xb,
                               nullptr);
    }
    return hipGetLastError();
}

template <int MT, bool GU, typename YT>
void launch_dot_rows(const WeightView& w, const ActPlanes& a, YT* y, int M, int64_t nout, int64_t up_off,
                     hipStream_t s) {
    const int K = (int)w.K;
    const size_t lds = lds_bytes(w.qtype, MT, K);
    if (w.qtype == 12) {
        const int64_t waves = (nout + 3) / 4;
        const dim3 grid((unsigned)((waves + 3) / 4), (unsigned)((M + MT - 1) / MT));
        hipLaunchKernelGGL((k_q8act_q4k<MT, GU, YT>), grid, dim3(256), lds, s, w.q, a.xq, a.xd, a.xb, y, M, nout, K,
                           up_off, nout, (uint32_t*)nullptr, (int8_t*)nullptr, (float*)nullptr, (int16_t*)nullptr);
        return;
    }
    // Q8_0 tiles: K ranges per tile as for the M = 1 GEMV (enough waves to fill the GPU)
    const int64_t tiles = (nout + 31) / 32;
    const int nch = (K / 32 + 7) / 8;
    const int ks = (tiles >= 2048 || nch < 2) ? 1 : ((tiles >= 1024 || nch < 4) ? 2 : 4);
    const int tpb = 4 / ks;
    const dim3 grid((unsigned)((tiles + tpb - 1) / tpb), (unsigned)((M + MT - 1) / MT));
    const int8_t* Q = reinterpret_cast<const int8_t*>(w.q);
    const uint16_t* D = reinterpret_cast<const uint16_t*>(w.aux);
    if (ks == 1)
        hipLaunchKernelGGL((k_q8act_q8_0<MT, 1, GU, YT>), grid, dim3(256), lds, s, Q, D, a.xq, a.xd, y, M, nout, K,
                           up_off, nout);
    else if (ks == 2)
        hipLaunchKernelGGL((k_q8act_q8_0<MT, 2, GU, YT>), grid, dim3(256), lds, s, Q, D, a.xq, a.xd, y, M, nout, K,
                           up_off, nout);
    else
        hipLaunchKernelGGL((k_q8act_q8_0<MT, 4, GU, YT>), grid, dim3(256), lds, s, Q, D, a.xq, a.xd, y, M, nout, K,
                           up_off, nout);
}

template <int MT, bool GU, typename YT>
void launch_dot(const WeightView& w, const ActPlanes& a, YT* y, int M, int64_t nout, int64_t up_off, hipStream_t s) {
    for (int64_t r0 = 0; r0 < M; r0 += kMaxGridY * MT) {
        const int mr = (int)(M - r0 < kMaxGridY * MT ? M - r0 : kMaxGridY * MT);
        launch_dot_rows<MT, GU, YT>(w, act_rows(a, w.qtype, w.K, r0), y + r0 * nout, mr, nout, up_off, s);
    }
}

template <bool GU, typename YT>
void launch_dot_mt(int mt, const WeightView& w, const ActPlanes& a, YT* y, int M, int64_t nout, int64_t up_off,
                   hipStream_t s) {
    switch (mt) {
        case 8: launch_dot<8, GU, YT>(w, a, y, M, nout, up_off, s); break;
        case 4: launch_dot<4, GU, YT>(w, a, y, M, nout, up_off, s); break;
        case 2: launch_dot<2, GU, YT>(w, a, y, M, nout, up_off, s); break;
        default: launch_dot<1, GU, YT>(w, a, y, M, nout, up_off, s); break;
    }
}

// the emitting gate/up; the arrival counters of a row chunk are left zero by
// its last blocks, so the next chunk reuses them
template <int MT, typename YT>
void launch_emit(const WeightView& w, const ActPlanes& a, YT* y, int M, int64_t nout, uint32_t* cnt,
                 const ActPlanes& o, hipStream_t s) {
    const int K = (int)w.K;
    const int64_t waves = (nout + 3) / 4;
    for (int64_t r0 = 0; r0 < M; r0 += kMaxGridY * MT) {
        const int mr = (int)(M - r0 < kMaxGridY * MT ? M - r0 : kMaxGridY * MT);
        const ActPlanes ac = act_rows(a, 12, K, r0), oc = act_rows(o, 12, nout, r0);
        const dim3 grid((unsigned)((waves + 3) / 4), (unsigned)((mr + MT - 1) / MT));
        hipLaunchKernelGGL((k_q8act_q4k<MT, true, YT, true>), grid, dim3(256), lds_bytes(12, MT, K), s, w.q, ac.xq,
                           ac.xd, ac.xb, y + r0 * nout, mr, nout, K, nout, nout, cnt, oc.xq, oc.xd, oc.xb);
    }
}

}  // namespace

size_t q8act_emit_counters(int64_t M, int64_t K, int64_t nout) {
    const int mt = pick_mt(12, M, (int)K);
    return (size_t)((M + mt - 1) / mt) * (size_t)(nout / 256);
}

hipError_t launch_q8act_dot_emit(const WeightView& w, const void* planes, void* y, bool yf32, int M, int64_t nout,
                                 uint32_t* counters, void* out_planes, hipStream_t s) {
    if (w.qtype != 12 || nout % 256) return hipErrorInvalidValue;
    const ActPlanes a = act_planes(12, const_cast<void*>(planes), M, w.K);
    const ActPlanes o = act_planes(12, out_planes, M, nout);
    const int mt = pick_mt(12, M, (int)w.K);
#define THQ_E(MT_)                                                                                                \
    (yf32 ? launch_emit<MT_, float>(w, a, static_cast<float*>(y), M, nout, counters, o, s)                       \
          : launch_emit<MT_, bf16_t>(w, a, static_cast<bf16_t*>(y), M, nout, counters, o, s))
    switch (mt) {
        case 8: THQ_E(8); break;
        case 4: THQ_E(4); break;
        case 2: THQ_E(2); break;
        default: THQ_E(1); break;
    }
#undef THQ_E
    return hipGetLastError();
}

bool q8act_supported(int qtype, int64_t K) { return lds_bytes(qtype, 1, (int)K) <= kLdsCap; }

size_t q8act_workspace_bytes(int qtype, int64_t M, int64_t K) {
    return align256((size_t)M * K) + align256((size_t)M * (K / (qtype == 12 ? 256 : 32)) * 4) +
           (qtype == 12 ? align256((size_t)M * (K / 32) * 2) : 0);
}

hipError_t launch_quantize_act(int qtype, const void* x, bool xf32, int64_t M, int64_t K, void* blocks,
                               hipStream_t s) {
    uint8_t* b = static_cast<uint8_t*>(blocks);
    return xf32 ? quant_act_t<float>(qtype, static_cast<const float*>(x), M, K, nullptr, b, s)
                : quant_act_t<bf16_t>(qtype, static_cast<const bf16_t*>(x), M, K, nullptr, b, s);
}

hipError_t launch_q8act_prepare(int qtype, const void* x, bool xf32, int64_t M, int64_t K, void* planes,
                                hipStream_t s) {
    const ActPlanes a = act_planes(qtype, planes, M, K);
    return xf32 ? quant_act_t<float>(qtype, static_cast<const float*>(x), M, K, &a, nullptr, s)
                : quant_act_t<bf16_t>(qtype, static_cast<const bf16_t*>(x), M, K, &a, nullptr, s);
}

hipError_t launch_q8act(const WeightView& w, const void* x, bool xf32, void* y, bool yf32, bool gu, int M,
                        int64_t nout, int64_t up_off, void* ws, hipStream_t s) {
    hipError_t e = launch_q8act_prepare(w.qtype, x, xf32, M, w.K, ws, s);
    if (e != hipSuccess) return e;
    return launch_q8act_dot(w, ws, y, yf32, gu, M, nout, up_off, s);
}

hipError_t launch_q8act_dot_tile(const TilePlan& p, const WeightView& w, const uint8_t* tiles, const void* planes,
                                 void* y, bool yf32, bool gu, int M, float* ws, uint32_t* cnt, hipStream_t s) {
    const ActPlanes a = act_planes(12, const_cast<void*>(planes), M, w.K);
    return launch_q8act_tile(p, w, tiles, a.xq, a.xd, a.xb, y, yf32, gu, M, ws, cnt, s);
}

hipError_t launch_q8act_tiled(const TilePlan& p, const WeightView& w, const uint8_t* tiles, const void* x, bool xf32,
                              void* y, bool yf32, bool gu, int M, void* planes, float* ws, uint32_t* cnt,
                              hipStream_t s) {
    hipError_t e = launch_q8act_prepare(12, x, xf32, M, w.K, planes, s);
    if (e != hipSuccess) return e;
    return launch_q8act_dot_tile(p, w, tiles, planes, y, yf32, gu, M, ws, cnt, s);
}

hipError_t launch_q8act_dot(const WeightView& w, const void* planes, void* y, bool yf32, bool gu, int M, int64_t nout,
                            int64_t up_off, hipStream_t s) {
    const ActPlanes a = act_planes(w.qtype, const_cast<void*>(planes), M, w.K);
    const int mt = pick_mt(w.qtype, M, (int)w.K);
    if (gu) {
        if (yf32) launch_dot_mt<true, float>(mt, w, a, static_cast<float*>(y), M, nout, up_off, s);
        else launch_dot_mt<true, bf16_t>(mt, w, a, static_cast<bf16_t*>(y), M, nout, up_off, s);
    } else {
        if (yf32) launch_dot_mt<false, float>(mt, w, a, static_cast<float*>(y), M, nout, up_off, s);
        else launch_dot_mt<false, bf16_t>(mt, w, a, static_cast<bf16_t*>(y), M, nout, up_off, s);
    }
    return hipGetLastError();
}

}  // namespace thq
