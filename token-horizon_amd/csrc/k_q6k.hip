// k_q6k.hip — Q6_K decode GEMV (M = 1, bf16 activations) for gfx950.
//
// Role: candle's QMatMul::forward at m = 1 over a Q6_K tensor, the type a
// Q4_K_M GGUF file keeps its output head and part of ffn_down / attn_v in
// (the loader engine/src/model.rs:526-562 hands them to quantized_qwen3).
// HBM-bound like the Q4_K GEMV: every weight byte is read once, x is staged
// in LDS once per block and held in registers across the rows a wave owns.
//
// Weights come from the QL / QH / SC / D planes, regrouped by 64-weight
// step (thq_dev.hpp, q6k_layout).  Lane map for one 4096-wide K chunk c: the
// lane takes step g = 64c + lane, i.e. 32 contiguous QL bytes, 16 QH bytes,
// one dword of 4 scales (one per 16-weight group) and its superblock's d, so
// the scale multiply happens once per 16 weights.
//
// Per 4 weights: 3 bit ops build four 6-bit codes in a dword, 2 v_perm put
// them under a constant 0x43 byte (bf16 0x43nn = 128 + code), 2
// v_dot2_f32_bf16 accumulate x * (128 + code); per scale group the offset is
// removed with the lane's sum of x: sum x * (code - 32) = dot - 160 * sum x.
#include "thq_dev.hpp"
#include "thq_kernels.hpp"
#include "thq_wave.hpp"

namespace thq {

struct Q6Planes {
    const uint8_t* ql;
    const uint8_t* qh;
    const uint8_t* sc;
    const uint16_t* d;
};

// one row's share of a lane: one 64-weight step in four scale groups of 16
struct Q6Row {
    uint32_t sc;   // the step's 4 scales, group G in byte G
    uint32_t d;    // the superblock's f16 d
    uint4 lo, hi;  // QL bytes 0..15 (weights t and t + 32), 16..31 (t + 16, t + 48)
    uint4 h;       // QH bytes 0..15 (2-bit fields of weights t, t+16, t+32, t+48)
};

__device__ __forceinline__ void q6_row_load(Q6Row& R, const Q6Planes& P, int64_t row, int K, int g) {
    const int nsb = K >> 8;
    // scales and d first: the in-order wait counters then release a row's
    // math as soon as its own bytes have landed
    R.sc = *reinterpret_cast<const uint32_t*>(P.sc + row * (K >> 4) + 4 * g);
    R.d = P.d[row * nsb + (g >> 2)];
    const uint8_t* ql = P.ql + row * (K >> 1) + 32 * g;
    R.lo = *reinterpret_cast<const uint4*>(ql);
    R.hi = *reinterpret_cast<const uint4*>(ql + 16);
    R.h = *reinterpret_cast<const uint4*>(P.qh + row * (K >> 2) + 16 * g);
}

// sum over the lane's 64 weights of x * w, w = (d * sc) * (code - 32); xq[G]
// holds the bf16 pairs of group G (weights 16G .. 16G + 15), sx[G] their sum
__device__ __forceinline__ float q6_row_dot(const Q6Row& R, const uint32_t (&xq)[4][8], const float (&sx)[4],
                                            float dlive) {
    const uint32_t C43 = 0x43434343u;
    const uint32_t lo[4] = {R.lo.x, R.lo.y, R.lo.z, R.lo.w};
    const uint32_t hi[4] = {R.hi.x, R.hi.y, R.hi.z, R.hi.w};
    const uint32_t hh[4] = {R.h.x, R.h.y, R.h.z, R.h.w};
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t A = lo[t], B = hi[t], H = hh[t];
        uint32_t c[4];
        c[0] = (A & 0x0F0F0F0Fu) | ((H & 0x03030303u) << 4);          // weights 4t .. 4t+3
        c[1] = (B & 0x0F0F0F0Fu) | ((H & 0x0C0C0C0Cu) << 2);          // 16 + 4t ..
        c[2] = ((A >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u);          // 32 + 4t ..
        c[3] = ((B >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u);   // 48 + 4t ..
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            // perm(C43, v, sel): bytes [v.b_i, 0x43, v.b_i+1, 0x43] = bf16 pair (128+q_i, 128+q_i+1)
            a[q] = dot2_bf16(__builtin_amdgcn_perm(C43, c[q], 0x04010400u), xq[q][2 * t], a[q]);
            a[q] = dot2_bf16(__builtin_amdgcn_perm(C43, c[q], 0x04030402u), xq[q][2 * t + 1], a[q]);
        }
    }
    const float s0 = (float)(int)(int8_t)R.sc, s1 = (float)(int)(int8_t)(R.sc >> 8);
    const float s2 = (float)(int)(int8_t)(R.sc >> 16), s3 = (float)(int)(int8_t)(R.sc >> 24);
    float p = s0 * __builtin_fmaf(-160.0f, sx[0], a[0]);
    p = __builtin_fmaf(s1, __builtin_fmaf(-160.0f, sx[1], a[1]), p);
    p = __builtin_fmaf(s2, __builtin_fmaf(-160.0f, sx[2], a[2]), p);
    p = __builtin_fmaf(s3, __builtin_fmaf(-160.0f, sx[3], a[3]), p);
    return (dlive * f16_to_f32((uint16_t)R.d)) * p;
}

// A block holds QPB row groups x KC waves; wave (group, chunk) takes its
// 4096-wide K chunk of the group's 4 rows (2 gate + 2 up rows in gate/up
// mode).  All loads are issued at entry: x first (so the wait before x goes
// to LDS covers only x), then the rows.  The chunks' row totals are summed in
// LDS in chunk order before the epilogue.  x is staged with 8 / QPB 16-B
// pieces per thread (K / 8 <= 512 * KC).
template <int KC, int QPB, bool GU, typename YT>
__global__ __launch_bounds__(64 * QPB * KC) void k_gemv1_q6k_bf16(Q6Planes P, const bf16_t* x, YT* __restrict__ y,
                                                                 int64_t nout, int K, int64_t up_off,
                                                                 int64_t ngroups, float* __restrict__ amv,
                                                                 uint32_t* __restrict__ ami) {
    static_assert(QPB == 2 || QPB == 4, "x staging uses two or four pieces per thread");
    extern __shared__ uint4 lds[];  // x (K bf16)
    __shared__ float red[QPB][KC][4];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int c = wv % KC, qb = wv / KC;
    const int64_t g = (int64_t)blockIdx.x * QPB + qb;
    const int nsb = K >> 8;
    const int nx = K >> 3, nt = 64 * QPB * KC;
    const int x0 = threadIdx.x, x1 = x0 + nt, x2 = x1 + nt, x3 = x2 + nt;
    const uint4 xv0 = reinterpret_cast<const uint4*>(x)[x0 < nx ? x0 : nx - 1];
    const uint4 xv1 = reinterpret_cast<const uint4*>(x)[x1 < nx ? x1 : nx - 1];
    uint4 xv2 = xv1, xv3 = xv1;
    if constexpr (QPB == 2) {
        xv2 = reinterpret_cast<const uint4*>(x)[x2 < nx ? x2 : nx - 1];
        xv3 = reinterpret_cast<const uint4*>(x)[x3 < nx ? x3 : nx - 1];
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    // lanes past K read step 0 and are masked to zero
    const bool live = 16 * c + (lane >> 2) < nsb;
    const int gs = live ? 64 * c + lane : 0;
    const int64_t base = GU ? 2 * g : 4 * g;
    Q6Row A0, A1, A2, A3;
    {
        auto row_of = [&](int r) -> int64_t {
            const int64_t o = GU ? base + (r >> 1) : base + r;  // output index of slot r
            return (g < ngroups && o < nout) ? slot_row<4, GU>(base, r, up_off) : 0;
        };
        q6_row_load(A0, P, row_of(0), K, gs);
        q6_row_load(A1, P, row_of(1), K, gs);
        q6_row_load(A2, P, row_of(2), K, gs);
        q6_row_load(A3, P, row_of(3), K, gs);
    }
    if (x0 < nx) lds[x0] = xv0;
    if (x1 < nx) lds[x1] = xv1;
    if constexpr (QPB == 2) {
        if (x2 < nx) lds[x2] = xv2;
        if (x3 < nx) lds[x3] = xv3;
    }
    __syncthreads();

    // the lane's activations: elements 64 gs .. 64 gs + 63, group G = 16 of them
    const uint32_t m = live ? 0xFFFFFFFFu : 0u;
    uint32_t xq[4][8];
    float sx[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint4* xp = lds + 8 * gs + 2 * q;
        const uint4 p0 = xp[0], p1 = xp[1];
        xq[q][0] = p0.x & m; xq[q][1] = p0.y & m; xq[q][2] = p0.z & m; xq[q][3] = p0.w & m;
        xq[q][4] = p1.x & m; xq[q][5] = p1.y & m; xq[q][6] = p1.z & m; xq[q][7] = p1.w & m;
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) t = dot2_bf16(xq[q][i], 0x3F803F80u, t);  // bf16 (1, 1)
        sx[q] = t;
    }
    const float dl = live ? 1.0f : 0.0f;  // a dead lane's d may be any f16, even inf
    const float acc[4] = {q6_row_dot(A0, xq, sx, dl), q6_row_dot(A1, xq, sx, dl), q6_row_dot(A2, xq, sx, dl),
                          q6_row_dot(A3, xq, sx, dl)};
    const float tot = reduce_slots<4>(acc, lane);
    if (!(lane & 15)) red[qb][c][slot_of_lane<4>(lane)] = tot;
    __syncthreads();
    constexpr int NO = GU ? 2 : 4;  // outputs per row group
    if (!GU && amv) {
        // fused argmax: the block's QPB * 4 outputs (summed over chunks exactly
        // as the stored path) reduce across wave 0's first lanes to one
        // (max, lowest index) partial
        static_assert(QPB * 4 <= 16, "one DPP row holds the block's outputs");
        if (threadIdx.x < 64) {
            const int64_t o = (int64_t)blockIdx.x * QPB * 4 + threadIdx.x;
            const bool own = threadIdx.x < QPB * 4;
            float v = -INFINITY;
            if (own && o < nout) {
                float a = 0.0f;
#pragma unroll
                for (int k = 0; k < KC; ++k) a += red[threadIdx.x >> 2][k][threadIdx.x & 3];
                v = amax_key(a);
            }
            uint32_t i = own ? (uint32_t)o : 0xFFFFFFFFu;
            amax_row16(v, i);
            if (threadIdx.x == 0) {
                amv[blockIdx.x] = v;
                ami[blockIdx.x] = i;
            }
        }
        return;
    }
    if (threadIdx.x < QPB * NO) {
        const int q2 = threadIdx.x / NO, p = threadIdx.x % NO;
        const int64_t o = (int64_t)NO * ((int64_t)blockIdx.x * QPB + q2) + p;
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int k = 0; k < KC; ++k) {
            a += red[q2][k][GU ? 2 * p : p];
            if (GU) b += red[q2][k][2 * p + 1];
        }
        if (o < nout) store_y<YT>(y + o, GU ? silu_mul(a, b) : a);
    }
}

template <int KC, int QPB, bool GU, typename YT>
static void q6_launch(const Q6Planes& P, const bf16_t* x, YT* y, int64_t nout, int K, int64_t up_off, hipStream_t s,
                      AmaxOut* am) {
    constexpr int NO = GU ? 2 : 4;
    const int64_t ngroups = (nout + NO - 1) / NO;
    const int64_t blocks = (ngroups + QPB - 1) / QPB;
    float* amv = nullptr;
    uint32_t* ami = nullptr;
    if (am) {  // one partial per block (M = 1)
        if (GU || blocks > am->ld) return;
        amv = am->v;
        ami = am->i;
        am->nb = blocks;
    }
    hipLaunchKernelGGL((k_gemv1_q6k_bf16<KC, QPB, GU, YT>), dim3((unsigned)blocks), dim3(64 * QPB * KC),
                       (size_t)K * 2, s, P, x, y, nout, K, up_off, ngroups, amv, ami);
}

template <bool GU, typename YT>
static hipError_t q6_dispatch(const Q6Planes& P, const bf16_t* x, YT* y, int64_t nout, int K, int64_t up_off,
                              hipStream_t s, AmaxOut* am) {
    switch ((K + 4095) / 4096) {
        case 1: q6_launch<1, 4, GU, YT>(P, x, y, nout, K, up_off, s, am); break;
        case 2: q6_launch<2, 2, GU, YT>(P, x, y, nout, K, up_off, s, am); break;
        case 3: q6_launch<3, 2, GU, YT>(P, x, y, nout, K, up_off, s, am); break;
        case 4: q6_launch<4, 2, GU, YT>(P, x, y, nout, K, up_off, s, am); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemv1_q6k(const WeightView& w, const void* x, void* y, bool yf32, bool gu, int64_t nout,
                            int64_t up_off, hipStream_t s, AmaxOut* am) {
    const int K = (int)w.K;
    if (w.qtype != 14 || K % 256 || K > 4 * 4096 || nout <= 0) return hipErrorInvalidValue;
    const Q6Layout L = q6k_layout(w.N, w.K);
    const Q6Planes P{w.q, w.q + L.qh, w.q + L.sc, reinterpret_cast<const uint16_t*>(w.q + L.d)};
    const bf16_t* xb = static_cast<const bf16_t*>(x);
    if (gu) return yf32 ? q6_dispatch<true, float>(P, xb, (float*)y, nout, K, up_off, s, am)
                        : q6_dispatch<true, bf16_t>(P, xb, (bf16_t*)y, nout, K, up_off, s, am);
    return yf32 ? q6_dispatch<false, float>(P, xb, (float*)y, nout, K, up_off, s, am)
                : q6_dispatch<false, bf16_t>(P, xb, (bf16_t*)y, nout, K, up_off, s, am);
}

}  // namespace thq
