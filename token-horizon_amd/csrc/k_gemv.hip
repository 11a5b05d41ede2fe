// k_gemv.hip — decode GEMV kernels (M = 1) for gfx950 and the exact generic
// fallback (any M <= 8, any alignment, f32 or bf16 activations).
//
// Role: the m = 1 projection of the reference (AffineQmvT,
// engine/src/quant_kernel.rs:2964-3140; candle QMatMul::forward at m = 1),
// here over GGUF Q4_K / Q8_0 weights.  HBM-bound: every weight byte is read
// once with 16-B loads, activations are held in registers and reused across
// the R rows a wave owns, and each row is reduced across the 64 lanes.
//
// Q4_K lane map (one 4096-wide K chunk per pass): lane = 4*s + p handles
// superblock s (0..15 of the chunk) and 64-element part p: bytes
// qs[32p .. 32p+32) hold elements 64p+i (low nibble, sub-block 2p) and
// 64p+32+i (high nibble, sub-block 2p+1).
#include "thq_dev.hpp"
#include "thq_kernels.hpp"
#include "thq_wave.hpp"

namespace thq {

// ------------------------------------------------------------------ Q4_K M=1, bf16 x
// Persistent: a fixed grid of waves walks "units" = (row quad, 4096-wide K
// chunk); each wave owns quads w, w + W, ... and all their chunks, and issues
// the loads of its next unit before computing the current one, so HBM
// streaming overlaps the VALU work.  With the row-quad layout a unit is nine
// contiguous 1-KB wave loads: eight nibble pieces (row r, half h) and the
// quad's transposed header dwords.  Gate/up: a unit holds the gate quad and
// the matching up quad (8 slots).  x and its per-lane sub-block sums come
// from LDS, staged once per block.
//
// Per 8 weights: 2 masks, 4 v_perm against a constant 0x43 byte (bf16 0x43nn
// = 128 + q), 4 v_dot2_f32_bf16; the 128 offset is removed with the lane's
// sum of x; d and dmin are assembled from the quad's header dwords with DPP.
template <bool GU>
struct Q4Unit {
    static constexpr int NQ = GU ? 2 : 1;
    uint4 nib[NQ][4][2];
    uint4 hdr[NQ];
};

// lane's 16-B offsets inside a row quad for chunk c (clamped to a real
// superblock: lanes past K multiply by zero activations)
template <bool GU>
__device__ __forceinline__ void q4k_unit_load(Q4Unit<GU>& U, const uint8_t* W, int64_t gq, int c,
                                              int64_t up_off, int nsb, int lane) {
    int s = 16 * c + (lane >> 2);
    const int li = s < nsb ? 16 * c * 4 + lane : (lane & 3);
    const int64_t qb = (int64_t)nsb * 576;
#pragma unroll
    for (int qi = 0; qi < Q4Unit<GU>::NQ; ++qi) {
        const uint8_t* g = W + (qi ? (gq + (up_off >> 2)) : gq) * qb + (int64_t)li * 16;
        // headers first: the in-order wait counters then let row r's math
        // start once its own two pieces have landed
        U.hdr[qi] = ld_stream16(g + (int64_t)nsb * 512);
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                U.nib[qi][r][h] = ld_stream16(g + (int64_t)r * nsb * 128 + (int64_t)h * nsb * 64);
    }
}

template <bool GU, bool AFF>
__device__ __forceinline__ void q4k_unit_compute(float (&acc)[GU ? 8 : 4], const Q4Unit<GU>& U,
                                                 const uint32_t (&xlo)[16], const uint32_t (&xhi)[16], float sxlo,
                                                 float sxhi) {
    const uint32_t C43 = 0x43434343u;
#pragma unroll
    for (int qi = 0; qi < Q4Unit<GU>::NQ; ++qi) {
        const uint32_t hq[4] = {U.hdr[qi].x, U.hdr[qi].y, U.hdr[qi].z, U.hdr[qi].w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint4 v0 = U.nib[qi][r][0], v1 = U.nib[qi][r][1];
            const uint32_t qw[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            float alo = 0.0f, ahi = 0.0f;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const uint32_t lo = qw[t] & 0x0F0F0F0Fu, hi = (qw[t] >> 4) & 0x0F0F0F0Fu;
                // perm(C43, v, sel): bytes [v.b_i, 0x43, v.b_i+1, 0x43] = bf16 pair (128+q_i, 128+q_i+1)
                alo = dot2_bf16(__builtin_amdgcn_perm(C43, lo, 0x04010400u), xlo[2 * t], alo);
                alo = dot2_bf16(__builtin_amdgcn_perm(C43, lo, 0x04030402u), xlo[2 * t + 1], alo);
                ahi = dot2_bf16(__builtin_amdgcn_perm(C43, hi, 0x04010400u), xhi[2 * t], ahi);
                ahi = dot2_bf16(__builtin_amdgcn_perm(C43, hi, 0x04030402u), xhi[2 * t + 1], ahi);
            }
            const uint32_t h = hq[r];
            if constexpr (AFF) {
                // affine group: sum x*w = scale * (a - 128 * sum x) + bias * sum x
                const float sc = aff_scale(h), bi = aff_bias(h), sx = sxlo + sxhi;
                const float a = __builtin_fmaf(sc, __builtin_fmaf(-128.0f, sx, alo + ahi), acc[4 * qi + r]);
                acc[4 * qi + r] = __builtin_fmaf(bi, sx, a);
                continue;
            }
            const uint32_t t0 = quad_bcast<0>(h), t1 = quad_bcast<1>(h);
            const uint32_t t2 = quad_bcast<2>(h), t3 = quad_bcast<3>(h);
            const float d = f16_to_f32((uint16_t)__builtin_amdgcn_perm(t1, t0, 0x0c0c0703u));
            const float dmin = f16_to_f32((uint16_t)__builtin_amdgcn_perm(t3, t2, 0x0c0c0703u));
            const float sc0 = (float)(h & 63u), m0 = (float)((h >> 6) & 63u);
            const float sc1 = (float)((h >> 12) & 63u), m1 = (float)((h >> 18) & 63u);
            // sum x*q = a - 128 * sum x, per sub-block; then d*sc and dmin*m
            const float dot = __builtin_fmaf(sc1, ahi, sc0 * alo);
            const float ssc = __builtin_fmaf(sc1, sxhi, sc0 * sxlo);
            const float smn = __builtin_fmaf(m1, sxhi, m0 * sxlo);
            float a = __builtin_fmaf(d, __builtin_fmaf(-128.0f, ssc, dot), acc[4 * qi + r]);
            acc[4 * qi + r] = __builtin_fmaf(-dmin, smn, a);
        }
    }
}

// 8-slot transposed reduction: lanes with (lane & 7) == 0 end with slot
// 4*(lane/32) + 2*((lane/16)%2) + (lane/8)%2
__device__ __forceinline__ float reduce_slots8(const float (&v)[8], int lane) {
    const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8;
    float k[4], k2[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) k[i] = (b5 ? v[4 + i] : v[i]) + __shfl_xor(b5 ? v[i] : v[4 + i], 32, 64);
#pragma unroll
    for (int i = 0; i < 2; ++i) k2[i] = (b4 ? k[2 + i] : k[i]) + __shfl_xor(b4 ? k[i] : k[2 + i], 16, 64);
    float t = (b3 ? k2[1] : k2[0]) + __shfl_xor(b3 ? k2[0] : k2[1], 8, 64);
    t += dpp_f<0xB1>(t);   // quad_perm [1,0,3,2]
    t += dpp_f<0x4E>(t);   // quad_perm [2,3,0,1]
    t += dpp_f<0x141>(t);  // row_half_mirror
    return t;
}

template <bool GU, typename YT>
__device__ __forceinline__ void q4k_unit_store(YT* __restrict__ y, int64_t gq, int64_t nout, int lane,
                                               const float (&acc)[GU ? 8 : 4]) {
    if constexpr (GU) {
        const float tot = reduce_slots8(acc, lane);
        const float u = __shfl_xor(tot, 32, 64);  // up slot = gate slot + 4
        if ((lane & 7) || (lane & 32)) return;
        const int64_t o = 4 * gq + ((lane >> 3) & 3);
        if (o < nout) store_y<YT>(y + o, silu_mul(tot, u));
    } else {
        const float tot = reduce_slots<4>(acc, lane);
        if (lane & 15) return;
        const int64_t o = 4 * gq + slot_of_lane<4>(lane);
        if (o < nout) store_y<YT>(y + o, tot);
    }
}

template <int KC, bool GU, bool AFF, typename YT>
__global__ __launch_bounds__(256) void k_gemv1_q4k_bf16(const uint8_t* __restrict__ W, const bf16_t* __restrict__ x,
                                                       YT* __restrict__ y, int64_t nout, int K, int64_t up_off,
                                                       int64_t nquads) {
    extern __shared__ uint4 lds[];  // x (K bf16)
    const int lane = threadIdx.x & 63;
    const int64_t nwaves = (int64_t)gridDim.x * (blockDim.x >> 6);
    const int64_t w = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int nsb = K >> 8;
    // units of this wave: quads w, w + nwaves, ... times KC chunks
    const int64_t nunits = (w < nquads ? (nquads - 1 - w) / nwaves + 1 : 0) * KC;

    Q4Unit<GU> A, B;
    if (nunits) q4k_unit_load<GU>(A, W, w, 0, up_off, nsb, lane);
    for (int i = threadIdx.x; i < (K >> 3); i += blockDim.x) lds[i] = reinterpret_cast<const uint4*>(x)[i];
    __syncthreads();
    if (!nunits) return;

    // this lane's activations for every chunk (bf16 pairs) and their sums
    uint32_t xlo[KC][16], xhi[KC][16];
    float sxlo[KC], sxhi[KC];
#pragma unroll
    for (int c = 0; c < KC; ++c) {
        const int s = 16 * c + (lane >> 2);
        float a0 = 0.0f, b0 = 0.0f;
        if (s < nsb) {
            const uint4* xp = lds + s * 32 + 8 * (lane & 3);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint4 p = xp[v], q = xp[4 + v];
                xlo[c][4 * v] = p.x; xlo[c][4 * v + 1] = p.y; xlo[c][4 * v + 2] = p.z; xlo[c][4 * v + 3] = p.w;
                xhi[c][4 * v] = q.x; xhi[c][4 * v + 1] = q.y; xhi[c][4 * v + 2] = q.z; xhi[c][4 * v + 3] = q.w;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                a0 = dot2_bf16(xlo[c][i], 0x3F803F80u, a0);  // bf16 (1, 1)
                b0 = dot2_bf16(xhi[c][i], 0x3F803F80u, b0);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) { xlo[c][i] = 0; xhi[c][i] = 0; }
        }
        sxlo[c] = a0;
        sxhi[c] = b0;
    }

    float acc[GU ? 8 : 4];
#pragma unroll
    for (int i = 0; i < (GU ? 8 : 4); ++i) acc[i] = 0.0f;
    // unit i = (quad w + (i / KC) * nwaves, chunk i % KC); walk it incrementally
    int64_t gq = w;
    int c = 0;
    auto advance = [&](int64_t& q, int& ch) {
        if (++ch == KC) { ch = 0; q += nwaves; }
    };
    auto finish = [&](const Q4Unit<GU>& U, int64_t q, int ch) {
        // KC is small: select the chunk's activations with a static switch
#pragma unroll
        for (int cc = 0; cc < KC; ++cc)
            if (cc == ch) q4k_unit_compute<GU, AFF>(acc, U, xlo[cc], xhi[cc], sxlo[cc], sxhi[cc]);
        if (ch == KC - 1) {
            q4k_unit_store<GU, YT>(y, q, nout, lane, acc);
#pragma unroll
            for (int j = 0; j < (GU ? 8 : 4); ++j) acc[j] = 0.0f;
        }
    };
    // two units per trip so the A/B register sets never need copying
    for (int64_t i = 0;; i += 2) {
        int64_t q1 = gq;
        int c1 = c;
        advance(q1, c1);
        if (i + 1 < nunits) q4k_unit_load<GU>(B, W, q1, c1, up_off, nsb, lane);
        finish(A, gq, c);
        if (i + 1 >= nunits) break;
        int64_t q2 = q1;
        int c2 = c1;
        advance(q2, c2);
        if (i + 2 < nunits) q4k_unit_load<GU>(A, W, q2, c2, up_off, nsb, lane);
        finish(B, q1, c1);
        if (i + 2 >= nunits) break;
        gq = q2;
        c = c2;
    }
}

// K-split one-shot variant for 4096 < K <= KC * 4096: a block holds QPB row
// quads x KC waves, wave (quad, chunk) loads its 4096-wide chunk of the quad
// at entry (after the block's x loads, as in the one-shot kernel) and the
// chunks' row totals are summed in LDS in chunk order before the epilogue.
// x is staged with 8 / QPB 16-B chunks per thread (K / 8 <= 512 * KC).
template <int KC, int QPB, bool GU, bool AFF, typename YT>
__global__ __launch_bounds__(64 * QPB * KC) void k_gemv1_q4k_bf16_ks(const uint8_t* W, const bf16_t* x,
                                                                    YT* __restrict__ y, int64_t nout, int K,
                                                                    int64_t up_off, int64_t nquads) {
    static_assert(QPB == 2 || QPB == 4, "x staging uses two or four chunks per thread");
    extern __shared__ uint4 lds[];  // x (K bf16)
    __shared__ float red[QPB][KC][8];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int c = wv % KC, qb = wv / KC;
    const int64_t gq = (int64_t)blockIdx.x * QPB + qb;
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
    Q4Unit<GU> A;
    q4k_unit_load<GU>(A, W, gq < nquads ? gq : nquads - 1, c, up_off, nsb, lane);
    if (x0 < nx) lds[x0] = xv0;
    if (x1 < nx) lds[x1] = xv1;
    if constexpr (QPB == 2) {
        if (x2 < nx) lds[x2] = xv2;
        if (x3 < nx) lds[x3] = xv3;
    }
    __syncthreads();
    const int s = 16 * c + (lane >> 2);
    uint32_t xlo[16], xhi[16];
    float sxlo = 0.0f, sxhi = 0.0f;
    if (s < nsb) {
        const uint4* xp = lds + s * 32 + 8 * (lane & 3);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint4 p = xp[v], q = xp[4 + v];
            xlo[4 * v] = p.x; xlo[4 * v + 1] = p.y; xlo[4 * v + 2] = p.z; xlo[4 * v + 3] = p.w;
            xhi[4 * v] = q.x; xhi[4 * v + 1] = q.y; xhi[4 * v + 2] = q.z; xhi[4 * v + 3] = q.w;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            sxlo = dot2_bf16(xlo[i], 0x3F803F80u, sxlo);  // bf16 (1, 1)
            sxhi = dot2_bf16(xhi[i], 0x3F803F80u, sxhi);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) { xlo[i] = 0; xhi[i] = 0; }
    }
    float acc[GU ? 8 : 4];
#pragma unroll
    for (int i = 0; i < (GU ? 8 : 4); ++i) acc[i] = 0.0f;
    q4k_unit_compute<GU, AFF>(acc, A, xlo, xhi, sxlo, sxhi);
    // per-chunk row totals: slots 0..3 (gate rows for GU), 4..7 (up rows)
    if constexpr (GU) {
        const float tot = reduce_slots8(acc, lane);
        if (!(lane & 7)) red[qb][c][4 * (lane >> 5) + 2 * ((lane >> 4) & 1) + ((lane >> 3) & 1)] = tot;
    } else {
        const float tot = reduce_slots<4>(acc, lane);
        if (!(lane & 15)) red[qb][c][slot_of_lane<4>(lane)] = tot;
    }
    __syncthreads();
    if (threadIdx.x < 4 * QPB) {
        const int q2 = threadIdx.x >> 2, r = threadIdx.x & 3;
        float g = 0.0f, u = 0.0f;
#pragma unroll
        for (int cc = 0; cc < KC; ++cc) {
            g += red[q2][cc][r];
            if (GU) u += red[q2][cc][r + 4];
        }
        const int64_t o = 4 * ((int64_t)blockIdx.x * QPB + q2) + r;
        if (o < nout) store_y<YT>(y + o, GU ? silu_mul(g, u) : g);
    }
}

// One-shot variant for K <= 4096: one wave per row quad, every load issued at
// entry, no second register set (so enough waves stay resident to keep the
// HBM queues full).  The block's x loads are issued before the weight loads:
// the wait before x goes to LDS then covers only x (vector-memory counters
// drain in order), so the block barrier does not hold the math back until
// every weight byte has landed, and each row's math starts as its data
// arrives.  W and x are not __restrict__ so that the compiler barrier keeps
// that order.
template <bool GU, bool AFF, bool FULL, typename YT>
__global__ __launch_bounds__(256) void k_gemv1_q4k_bf16_1s(const uint8_t* W, const bf16_t* x, YT* __restrict__ y,
                                                          int64_t nout, int K, int64_t up_off, int64_t nquads,
                                                          float* __restrict__ amv, uint32_t* __restrict__ ami) {
    extern __shared__ uint4 lds[];  // x (K bf16)
    const int lane = threadIdx.x & 63;
    const int64_t gq = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int nsb = K >> 8;
    // 16-B chunks of x: two per thread (K / 8 <= 512)
    const int nx = K >> 3;
    const int c0 = threadIdx.x, c1 = threadIdx.x + 256;
    const uint4 xv0 = reinterpret_cast<const uint4*>(x)[c0 < nx ? c0 : nx - 1];
    const uint4 xv1 = reinterpret_cast<const uint4*>(x)[c1 < nx ? c1 : nx - 1];
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    Q4Unit<GU> A;  // unconditional (clamped quad) so the wait counts stay exact
    q4k_unit_load<GU>(A, W, gq < nquads ? gq : nquads - 1, 0, up_off, nsb, lane);
    if (c0 < nx) lds[c0] = xv0;
    if (c1 < nx) lds[c1] = xv1;
    __syncthreads();
    if (gq >= nquads) return;
    // K = 4096 (FULL): every lane has a superblock; otherwise lanes past K
    // read a valid one and mask it to zero (branch-free either way)
    const int s = lane >> 2;
    const uint32_t live = (FULL || s < nsb) ? 0xFFFFFFFFu : 0u;
    const uint4* xp = lds + ((FULL || s < nsb) ? s : 0) * 32 + 8 * (lane & 3);
    uint32_t xlo[16], xhi[16];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const uint4 p = xp[v], q = xp[4 + v];
        xlo[4 * v] = p.x & live; xlo[4 * v + 1] = p.y & live; xlo[4 * v + 2] = p.z & live; xlo[4 * v + 3] = p.w & live;
        xhi[4 * v] = q.x & live; xhi[4 * v + 1] = q.y & live; xhi[4 * v + 2] = q.z & live; xhi[4 * v + 3] = q.w & live;
    }
    float sxlo = 0.0f, sxhi = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        sxlo = dot2_bf16(xlo[i], 0x3F803F80u, sxlo);  // bf16 (1, 1)
        sxhi = dot2_bf16(xhi[i], 0x3F803F80u, sxhi);
    }
    float acc[GU ? 8 : 4];
#pragma unroll
    for (int i = 0; i < (GU ? 8 : 4); ++i) acc[i] = 0.0f;
    q4k_unit_compute<GU, AFF>(acc, A, xlo, xhi, sxlo, sxhi);
    if constexpr (!GU) {
        if (amv) {
            // fused argmax: one (max, lowest index) partial per row quad; the
            // quad's outputs 4gq + s sit in lanes 16s after the slot reduction
            const float tot = reduce_slots<4>(acc, lane);
            const int64_t o = 4 * gq + slot_of_lane<4>(lane);
            float v = o < nout ? amax_key(tot) : -INFINITY;
            uint32_t i = (uint32_t)o;
            // every lane of a 16-lane group holds its slot's total: combine
            // the groups (lanes 0, 16, 32, 48 meet through xor 16 and 32)
#pragma unroll
            for (int off = 16; off <= 32; off <<= 1) {
                const float v2 = __shfl_xor(v, off, 64);
                const uint32_t i2 = __shfl_xor(i, off, 64);
                if (v2 > v || (v2 == v && i2 < i)) {
                    v = v2;
                    i = i2;
                }
            }
            if (lane == 0) {
                amv[gq] = v;
                ami[gq] = i;
            }
            return;
        }
    }
    q4k_unit_store<GU, YT>(y, gq, nout, lane, acc);
}

// ------------------------------------------------------------------ Q4_K M = 2..4, bf16 x
// The one-shot kernel with MR activation rows (K <= 4096): every weight byte
// is still read once per call, and each nibble pair's v_perm (bf16 128 + q)
// is built once and shared by the MR rows' v_dot2.  Rows m >= M are staged
// from row M-1 (in bounds) and never stored.
template <bool GU, bool AFF, int MR>
__device__ __forceinline__ void q4k_unit_compute_rows(float (&acc)[MR][GU ? 8 : 4], const Q4Unit<GU>& U,
                                                      const uint32_t (&xlo)[MR][16], const uint32_t (&xhi)[MR][16],
                                                      const float (&sxlo)[MR], const float (&sxhi)[MR]) {
    const uint32_t C43 = 0x43434343u;
#pragma unroll
    for (int qi = 0; qi < Q4Unit<GU>::NQ; ++qi) {
        const uint32_t hq[4] = {U.hdr[qi].x, U.hdr[qi].y, U.hdr[qi].z, U.hdr[qi].w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint4 v0 = U.nib[qi][r][0], v1 = U.nib[qi][r][1];
            const uint32_t qw[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            float alo[MR], ahi[MR];
#pragma unroll
            for (int m = 0; m < MR; ++m) alo[m] = ahi[m] = 0.0f;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const uint32_t lo = qw[t] & 0x0F0F0F0Fu, hi = (qw[t] >> 4) & 0x0F0F0F0Fu;
                const uint32_t p0 = __builtin_amdgcn_perm(C43, lo, 0x04010400u);
                const uint32_t p1 = __builtin_amdgcn_perm(C43, lo, 0x04030402u);
                const uint32_t p2 = __builtin_amdgcn_perm(C43, hi, 0x04010400u);
                const uint32_t p3 = __builtin_amdgcn_perm(C43, hi, 0x04030402u);
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    alo[m] = dot2_bf16(p0, xlo[m][2 * t], alo[m]);
                    alo[m] = dot2_bf16(p1, xlo[m][2 * t + 1], alo[m]);
                    ahi[m] = dot2_bf16(p2, xhi[m][2 * t], ahi[m]);
                    ahi[m] = dot2_bf16(p3, xhi[m][2 * t + 1], ahi[m]);
                }
            }
            const uint32_t h = hq[r];
            if constexpr (AFF) {
                const float sc = aff_scale(h), bi = aff_bias(h);
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    const float sx = sxlo[m] + sxhi[m];
                    const float a = __builtin_fmaf(sc, __builtin_fmaf(-128.0f, sx, alo[m] + ahi[m]), acc[m][4 * qi + r]);
                    acc[m][4 * qi + r] = __builtin_fmaf(bi, sx, a);
                    asm volatile("" : "+v"(acc[m][4 * qi + r]));
                }
                __builtin_amdgcn_sched_barrier(0);
                continue;
            }
            const uint32_t t0 = quad_bcast<0>(h), t1 = quad_bcast<1>(h);
            const uint32_t t2 = quad_bcast<2>(h), t3 = quad_bcast<3>(h);
            const float d = f16_to_f32((uint16_t)__builtin_amdgcn_perm(t1, t0, 0x0c0c0703u));
            const float dmin = f16_to_f32((uint16_t)__builtin_amdgcn_perm(t3, t2, 0x0c0c0703u));
            const float sc0 = (float)(h & 63u), m0 = (float)((h >> 6) & 63u);
            const float sc1 = (float)((h >> 12) & 63u), m1 = (float)((h >> 18) & 63u);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const float dot = __builtin_fmaf(sc1, ahi[m], sc0 * alo[m]);
                const float ssc = __builtin_fmaf(sc1, sxhi[m], sc0 * sxlo[m]);
                const float smn = __builtin_fmaf(m1, sxhi[m], m0 * sxlo[m]);
                const float a = __builtin_fmaf(d, __builtin_fmaf(-128.0f, ssc, dot), acc[m][4 * qi + r]);
                acc[m][4 * qi + r] = __builtin_fmaf(-dmin, smn, a);
            }
            // one weight row at a time: left free, the compiler builds every row's
            // perms up front (hundreds of VGPRs, occupancy 1)
#pragma unroll
            for (int m = 0; m < MR; ++m) asm volatile("" : "+v"(acc[m][4 * qi + r]));
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

template <int MR, bool GU, bool AFF, bool FULL, typename YT>
__global__ __launch_bounds__(256) void k_gemv_q4k_bf16_rows(const uint8_t* W, const bf16_t* x, YT* __restrict__ y,
                                                           int M, int64_t nout, int K, int64_t up_off,
                                                           int64_t nquads) {
    static_assert(MR == 2 || MR == 4, "two or four activation rows");
    extern __shared__ uint4 lds[];  // x rows (MR x K bf16)
    const int lane = threadIdx.x & 63;
    const int64_t gq = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int nsb = K >> 8;
    const int nx = K >> 3;
    const int c0 = threadIdx.x < nx ? threadIdx.x : nx - 1;
    const int c1 = threadIdx.x + 256 < nx ? threadIdx.x + 256 : nx - 1;
    const uint4* xg = reinterpret_cast<const uint4*>(x);
    const int r1 = 1 < M ? 1 : M - 1, r2 = 2 < M ? 2 : M - 1, r3 = 3 < M ? 3 : M - 1;
    // x loads first (named registers: arrays live across the compiler barrier spill)
    const uint4 xa0 = xg[c0], xa1 = xg[c1];
    const uint4 xb0 = xg[r1 * nx + c0], xb1 = xg[r1 * nx + c1];
    uint4 xc0 = xb0, xc1 = xb1, xd0 = xb0, xd1 = xb1;
    if constexpr (MR == 4) {
        xc0 = xg[r2 * nx + c0];
        xc1 = xg[r2 * nx + c1];
        xd0 = xg[r3 * nx + c0];
        xd1 = xg[r3 * nx + c1];
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    Q4Unit<GU> A;
    q4k_unit_load<GU>(A, W, gq < nquads ? gq : nquads - 1, 0, up_off, nsb, lane);
    const bool w0 = threadIdx.x < nx, w1 = threadIdx.x + 256 < nx;
    if (w0) { lds[threadIdx.x] = xa0; lds[nx + threadIdx.x] = xb0; }
    if (w1) { lds[threadIdx.x + 256] = xa1; lds[nx + threadIdx.x + 256] = xb1; }
    if constexpr (MR == 4) {
        if (w0) { lds[2 * nx + threadIdx.x] = xc0; lds[3 * nx + threadIdx.x] = xd0; }
        if (w1) { lds[2 * nx + threadIdx.x + 256] = xc1; lds[3 * nx + threadIdx.x + 256] = xd1; }
    }
    __syncthreads();
    if (gq >= nquads) return;
    const int s = lane >> 2;
    const uint32_t live = (FULL || s < nsb) ? 0xFFFFFFFFu : 0u;
    const int xoff = ((FULL || s < nsb) ? s : 0) * 32 + 8 * (lane & 3);
    uint32_t xlo[MR][16], xhi[MR][16];
    float sxlo[MR], sxhi[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const uint4* xp = lds + m * nx + xoff;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint4 p = xp[v], q = xp[4 + v];
            xlo[m][4 * v] = p.x & live; xlo[m][4 * v + 1] = p.y & live;
            xlo[m][4 * v + 2] = p.z & live; xlo[m][4 * v + 3] = p.w & live;
            xhi[m][4 * v] = q.x & live; xhi[m][4 * v + 1] = q.y & live;
            xhi[m][4 * v + 2] = q.z & live; xhi[m][4 * v + 3] = q.w & live;
        }
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            a = dot2_bf16(xlo[m][i], 0x3F803F80u, a);  // bf16 (1, 1)
            b = dot2_bf16(xhi[m][i], 0x3F803F80u, b);
        }
        sxlo[m] = a;
        sxhi[m] = b;
    }
    float acc[MR][GU ? 8 : 4];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int i = 0; i < (GU ? 8 : 4); ++i) acc[m][i] = 0.0f;
    q4k_unit_compute_rows<GU, AFF, MR>(acc, A, xlo, xhi, sxlo, sxhi);
#pragma unroll
    for (int m = 0; m < MR; ++m)
        if (m < M) q4k_unit_store<GU, YT>(y + (int64_t)m * nout, gq, nout, lane, acc[m]);
}

// K-split variant of the row kernel for 4096 < K <= 16384 and two activation
// rows: the block and chunk structure of k_gemv1_q4k_bf16_ks with QPB = 2
// row quads, both rows' x staged in LDS (4 pieces per thread per row).
template <int KC, bool GU, bool AFF, typename YT>
__global__ __launch_bounds__(128 * KC) void k_gemv_q4k_bf16_ks_rows(const uint8_t* W, const bf16_t* x,
                                                                   YT* __restrict__ y, int M, int64_t nout, int K,
                                                                   int64_t up_off, int64_t nquads) {
    constexpr int QPB = 2, MR = 2;
    extern __shared__ uint4 lds[];  // x rows (2 x K bf16)
    __shared__ float red[QPB][KC][MR][8];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int c = wv % KC, qb = wv / KC;
    const int64_t gq = (int64_t)blockIdx.x * QPB + qb;
    const int nsb = K >> 8;
    const int nx = K >> 3, nt = 64 * QPB * KC;
    const int i0 = threadIdx.x, i1 = i0 + nt, i2 = i1 + nt, i3 = i2 + nt;
    const int j0 = i0 < nx ? i0 : nx - 1, j1 = i1 < nx ? i1 : nx - 1;
    const int j2 = i2 < nx ? i2 : nx - 1, j3 = i3 < nx ? i3 : nx - 1;
    const uint4* xg = reinterpret_cast<const uint4*>(x);
    const int r1 = M > 1 ? nx : 0;  // second row (row 0 again when M == 1)
    const uint4 xa0 = xg[j0], xa1 = xg[j1], xa2 = xg[j2], xa3 = xg[j3];
    const uint4 xb0 = xg[r1 + j0], xb1 = xg[r1 + j1], xb2 = xg[r1 + j2], xb3 = xg[r1 + j3];
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    Q4Unit<GU> A;
    q4k_unit_load<GU>(A, W, gq < nquads ? gq : nquads - 1, c, up_off, nsb, lane);
    if (i0 < nx) { lds[i0] = xa0; lds[nx + i0] = xb0; }
    if (i1 < nx) { lds[i1] = xa1; lds[nx + i1] = xb1; }
    if (i2 < nx) { lds[i2] = xa2; lds[nx + i2] = xb2; }
    if (i3 < nx) { lds[i3] = xa3; lds[nx + i3] = xb3; }
    __syncthreads();
    const int s = 16 * c + (lane >> 2);
    const uint32_t live = s < nsb ? 0xFFFFFFFFu : 0u;
    const int xoff = (s < nsb ? s : 0) * 32 + 8 * (lane & 3);
    uint32_t xlo[MR][16], xhi[MR][16];
    float sxlo[MR], sxhi[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const uint4* xp = lds + m * nx + xoff;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint4 p = xp[v], q = xp[4 + v];
            xlo[m][4 * v] = p.x & live; xlo[m][4 * v + 1] = p.y & live;
            xlo[m][4 * v + 2] = p.z & live; xlo[m][4 * v + 3] = p.w & live;
            xhi[m][4 * v] = q.x & live; xhi[m][4 * v + 1] = q.y & live;
            xhi[m][4 * v + 2] = q.z & live; xhi[m][4 * v + 3] = q.w & live;
        }
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            a = dot2_bf16(xlo[m][i], 0x3F803F80u, a);  // bf16 (1, 1)
            b = dot2_bf16(xhi[m][i], 0x3F803F80u, b);
        }
        sxlo[m] = a;
        sxhi[m] = b;
    }
    float acc[MR][GU ? 8 : 4];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int i = 0; i < (GU ? 8 : 4); ++i) acc[m][i] = 0.0f;
    q4k_unit_compute_rows<GU, AFF, MR>(acc, A, xlo, xhi, sxlo, sxhi);
    // per-chunk row totals: slots 0..3 (gate rows for GU), 4..7 (up rows)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        if constexpr (GU) {
            const float tot = reduce_slots8(acc[m], lane);
            if (!(lane & 7)) red[qb][c][m][4 * (lane >> 5) + 2 * ((lane >> 4) & 1) + ((lane >> 3) & 1)] = tot;
        } else {
            const float tot = reduce_slots<4>(acc[m], lane);
            if (!(lane & 15)) red[qb][c][m][slot_of_lane<4>(lane)] = tot;
        }
    }
    __syncthreads();
    if (threadIdx.x < 4 * QPB * MR) {
        const int m = threadIdx.x / (4 * QPB), q2 = (threadIdx.x >> 2) % QPB, r = threadIdx.x & 3;
        float g = 0.0f, u = 0.0f;
#pragma unroll
        for (int cc = 0; cc < KC; ++cc) {
            g += red[q2][cc][m][r];
            if (GU) u += red[q2][cc][m][r + 4];
        }
        const int64_t o = 4 * ((int64_t)blockIdx.x * QPB + q2) + r;
        if (m < M && o < nout) store_y<YT>(y + (int64_t)m * nout + o, GU ? silu_mul(g, u) : g);
    }
}

// ------------------------------------------------------------------ Q4_K M=1, f32 x
template <int KC, int R, bool GU, bool AFF, typename YT>
__global__ __launch_bounds__(256) void k_gemv1_q4k_f32(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                      YT* __restrict__ y, int64_t nout, int K, int64_t up_off) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t base = wave * (GU ? R / 2 : R);
    if (base >= nout) return;
    const int nsb = K >> 8;
    const int sl = lane >> 2, part = lane & 3;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
        const int s = 16 * c + sl;
        if (s >= nsb) continue;
        float xl[32], xh[32];
        const float4* xp = reinterpret_cast<const float4*>(x + (int64_t)s * 256 + 64 * part);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const float4 a = xp[v], b = xp[8 + v];
            xl[4 * v] = a.x; xl[4 * v + 1] = a.y; xl[4 * v + 2] = a.z; xl[4 * v + 3] = a.w;
            xh[4 * v] = b.x; xh[4 * v + 1] = b.y; xh[4 * v + 2] = b.z; xh[4 * v + 3] = b.w;
        }
        float sxl = 0.0f, sxh = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) { sxl += xl[i]; sxh += xh[i]; }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            int64_t row = slot_row<R, GU>(base, r, up_off);
            const bool ok = GU ? (base + (r >> 1) < nout) : (row < nout);
            if (!ok) row = GU ? up_off * (r & 1) : 0;
            uint4 h;
            h.x = *reinterpret_cast<const uint32_t*>(W + q4k_hdword(row, nsb, s, 0));
            h.y = *reinterpret_cast<const uint32_t*>(W + q4k_hdword(row, nsb, s, 1));
            h.z = *reinterpret_cast<const uint32_t*>(W + q4k_hdword(row, nsb, s, 2));
            h.w = *reinterpret_cast<const uint32_t*>(W + q4k_hdword(row, nsb, s, 3));
            const uint4 a4 = *reinterpret_cast<const uint4*>(W + q4k_piece(row, nsb, s, 0, part));
            const uint4 b4 = *reinterpret_cast<const uint4*>(W + q4k_piece(row, nsb, s, 1, part));
            const uint32_t qw[8] = {a4.x, a4.y, a4.z, a4.w, b4.x, b4.y, b4.z, b4.w};
            float dl = 0.0f, dh = 0.0f;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    dl = __builtin_fmaf((float)((qw[t] >> (8 * b)) & 0xF), xl[4 * t + b], dl);
                    dh = __builtin_fmaf((float)((qw[t] >> (8 * b + 4)) & 0xF), xh[4 * t + b], dh);
                }
            }
            if constexpr (AFF) {
                const uint32_t hw = part == 0 ? h.x : (part == 1 ? h.y : (part == 2 ? h.z : h.w));
                acc[r] = __builtin_fmaf(aff_scale(hw), dl + dh, acc[r]);
                acc[r] = __builtin_fmaf(aff_bias(hw), sxl + sxh, acc[r]);
            } else {
                uint32_t sc0, m0, sc1, m1;
                q4k_hdr_sm(h, 2 * part, sc0, m0);
                q4k_hdr_sm(h, 2 * part + 1, sc1, m1);
                const float d = q4k_hdr_d(h), dmin = q4k_hdr_dmin(h);
                acc[r] = __builtin_fmaf(d, (float)sc0 * dl + (float)sc1 * dh, acc[r]);
                acc[r] = __builtin_fmaf(-dmin, (float)m0 * sxl + (float)m1 * sxh, acc[r]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
    write_rows<R, GU, YT>(y, base, nout, acc);
}

// ------------------------------------------------------------------ Q8_0 M=1
// Tile planes (thq_dev.hpp, q8t_q / q8t_d).  A wave takes one 32-row tile
// (outputs 32t .. 32t + 31; gate/up: the gate rows and the up rows of those
// outputs) over a range of 256-wide chunks and streams it: per chunk eight
// contiguous 1-KB loads (block b: lane (n, g) gets row n's bytes 16g ..
// 16g + 15) and one 16-B load of row n's eight scales.  A block's 4 waves are
// TPB = 4 / KS tiles x KS ranges of K (KS > 1 when there are too few tiles to
// fill the GPU); x is staged once per block in LDS with the sums of each
// 16-value run, and each lane reads its row's 16 values per block (one
// address per lane half: a broadcast).  u = q ^ 0x80 is the unsigned byte
// q + 128: bf16 x meets bf16(u) (exact) pairs in v_dot2_f32_bf16, f32 x
// v_cvt_f32_ubyte values in f32 fma; the 128 offset is removed with the sum.
// The two lanes of a row and the KS ranges are summed in that order at the
// end (LDS).  Fused argmax: one (max, lowest index) partial per block.
template <typename XT>
struct Q8TX;
template <>
struct Q8TX<bf16_t> {
    uint32_t v[8];
};
template <>
struct Q8TX<float> {
    float v[16];
};
template <typename XT>
__device__ __forceinline__ void q8t_xload(Q8TX<XT>& X, const XT* p) {
    if constexpr (sizeof(XT) == 2) {
        const uint4 a = *reinterpret_cast<const uint4*>(p);
        const uint4 b = *reinterpret_cast<const uint4*>(p + 8);
        X.v[0] = a.x; X.v[1] = a.y; X.v[2] = a.z; X.v[3] = a.w;
        X.v[4] = b.x; X.v[5] = b.y; X.v[6] = b.z; X.v[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 f = *reinterpret_cast<const float4*>(p + 4 * i);
            X.v[4 * i] = f.x; X.v[4 * i + 1] = f.y; X.v[4 * i + 2] = f.z; X.v[4 * i + 3] = f.w;
        }
    }
}
__device__ __forceinline__ float q8_dot16(const uint4& q, const Q8TX<bf16_t>& X) {
    const uint32_t u[4] = {q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u, q.w ^ 0x80808080u};
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        s = dot2_bf16(pack_bf16x2(ubyte_f32<0>(u[t]), ubyte_f32<1>(u[t])), X.v[2 * t], s);
        s = dot2_bf16(pack_bf16x2(ubyte_f32<2>(u[t]), ubyte_f32<3>(u[t])), X.v[2 * t + 1], s);
    }
    return s;
}
__device__ __forceinline__ float q8_dot16(const uint4& q, const Q8TX<float>& X) {
    const uint32_t u[4] = {q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u, q.w ^ 0x80808080u};
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        s = __builtin_fmaf(ubyte_f32<0>(u[t]), X.v[4 * t], s);
        s = __builtin_fmaf(ubyte_f32<1>(u[t]), X.v[4 * t + 1], s);
        s = __builtin_fmaf(ubyte_f32<2>(u[t]), X.v[4 * t + 2], s);
        s = __builtin_fmaf(ubyte_f32<3>(u[t]), X.v[4 * t + 3], s);
    }
    return s;
}
// one chunk of one weight row set: 8 block pieces and the row's 8 scales
struct Q8TChunk {
    uint4 q[8];
    uint4 d;
};

constexpr int Q8T_KMAX = 8192;  // x staged in LDS: K <= 8192

template <int KS, bool FULL, bool GU, typename XT, typename YT>
__global__ __launch_bounds__(256) void k_gemv1_q8(const int8_t* __restrict__ Q, const uint16_t* __restrict__ D,
                                                 const XT* __restrict__ x, YT* __restrict__ y, int64_t nout, int K,
                                                 int64_t up_off, float* __restrict__ amv, uint32_t* __restrict__ ami) {
    constexpr int TPB = 4 / KS;  // tiles per block
    constexpr int R = GU ? 2 : 1;
    __shared__ __attribute__((aligned(16))) XT xs[Q8T_KMAX];
    __shared__ float s16[Q8T_KMAX / 16];
    __shared__ float red[KS > 1 ? KS - 1 : 1][TPB][32][R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 31, g = lane >> 5;
    const int ti = wave % TPB, ks = wave / TPB;
    const int64_t tile = (int64_t)blockIdx.x * TPB + ti;
    const int64_t o = tile * 32 + n;           // this lane's output
    const bool live = o < nout;
    const int64_t nb = K >> 5;
    const int nch = (int)((nb + 7) >> 3);
    const int cpk = (nch + KS - 1) / KS;
    const int c0 = ks * cpk, c1 = c0 + cpk < nch ? c0 + cpk : nch;
    // rows of this lane (padding rows of the last tile read zero weights)
    int64_t rows[R];
    rows[0] = GU ? (live ? o : 0) : o;
    if constexpr (GU) rows[R - 1] = live ? o + up_off : 0;
    const int8_t* pq[R];
    const uint16_t* pd[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        pq[r] = Q + q8t_q(rows[r], nb, 0, g);
        pd[r] = D + q8t_d(rows[r], nb, 0);
    }
    auto load = [&](Q8TChunk (&C)[R], int c) {
        // blocks in chunk c (FULL: K % 256 == 0, every chunk whole)
        const int nbc = FULL ? 8 : ((int)(nb - 8 * (int64_t)c) < 8 ? (int)(nb - 8 * (int64_t)c) : 8);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            C[r].d = *reinterpret_cast<const uint4*>(pd[r] + (int64_t)c * 256);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                C[r].q[j] = j < nbc ? *reinterpret_cast<const uint4*>(pq[r] + ((int64_t)c * 8 + j) * 1024)
                                    : make_uint4(0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u);
        }
    };
    Q8TChunk cur[R];
    if (c0 < c1) load(cur, c0);
    // stage x (its loads wait behind the first chunk's: counters drain in order)
    // and the sum of each 16-value run: 2 (bf16) or 4 (f32) threads' pieces,
    // combined by DPP within the lane pair / quad (K % 32 == 0 keeps them whole)
    if constexpr (sizeof(XT) == 2) {
        for (int i = 8 * threadIdx.x; i < K; i += 8 * 256) {
            const uint4 v = *reinterpret_cast<const uint4*>(x + i);
            *reinterpret_cast<uint4*>(&xs[i]) = v;
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            float t = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) t += bf16_to_f32(w[e] & 0xFFFFu) + bf16_to_f32(w[e] >> 16);
            t += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(t), 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
            if ((threadIdx.x & 1) == 0) s16[i >> 4] = t;
        }
    } else {
        for (int i = 4 * threadIdx.x; i < K; i += 4 * 256) {
            const float4 v = *reinterpret_cast<const float4*>(x + i);
            *reinterpret_cast<float4*>(&xs[i]) = v;
            float t = (v.x + v.y) + (v.z + v.w);
            t += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(t), 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
            t += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(t), 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
            if ((threadIdx.x & 3) == 0) s16[i >> 4] = t;
        }
    }
    __syncthreads();

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    // each chunk's math, then the next chunk's loads into the same registers
    // (the compiler issues them ahead where registers allow; measured faster
    // than an explicit second buffer)
    for (int c = c0; c < c1; ++c) {
        const int nbc = FULL ? 8 : ((int)(nb - 8 * (int64_t)c) < 8 ? (int)(nb - 8 * (int64_t)c) : 8);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (j < nbc) {
                const int64_t k0 = (8 * (int64_t)c + j) * 32 + 16 * g;
                Q8TX<XT> X;
                q8t_xload<XT>(X, &xs[k0]);
                const float sx = s16[k0 >> 4];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint32_t dw = j < 2 ? cur[r].d.x : (j < 4 ? cur[r].d.y : (j < 6 ? cur[r].d.z : cur[r].d.w));
                    const float d = f16_to_f32((uint16_t)((j & 1) ? (dw >> 16) : dw));
                    acc[r] = __builtin_fmaf(d, __builtin_fmaf(-128.0f, sx, q8_dot16(cur[r].q[j], X)), acc[r]);
                }
            }
        }
        if (c + 1 < c1) load(cur, c + 1);
    }
    // the row's two lane halves, then the K ranges in order
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] += __shfl_xor(acc[r], 32, 64);
    if constexpr (KS > 1) {
        if (ks > 0 && g == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) red[ks - 1][ti][n][r] = acc[r];
        }
        __syncthreads();
        if (ks == 0) {
#pragma unroll
            for (int k = 0; k < KS - 1; ++k)
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r] += red[k][ti][n][r];
        }
    }
    if (!GU && amv) {
        // one (max, lowest index) partial per block: a scan from (-inf, o0)
        // over the block's outputs (NaN never wins, ties keep the lower index)
        __shared__ float amx[TPB];
        __shared__ uint32_t amn[TPB];
        float v = live ? acc[0] : -INFINITY;
        uint32_t i = (uint32_t)o;
        if (!(v > -INFINITY)) {
            v = -INFINITY;
            i = 0xFFFFFFFFu;
        }
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) {
            const float v2 = __shfl_xor(v, off, 64);
            const uint32_t i2 = __shfl_xor(i, off, 64);
            if (v2 > v || (v2 == v && i2 < i)) {
                v = v2;
                i = i2;
            }
        }
        if (ks == 0 && lane == 0) {
            amx[ti] = v;
            amn[ti] = i;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float bv = -INFINITY;
            uint32_t bi = (uint32_t)((int64_t)blockIdx.x * TPB * 32);
            for (int t = 0; t < TPB; ++t)
                if (amx[t] > bv || (amx[t] == bv && amx[t] > -INFINITY && amn[t] < bi)) {
                    bv = amx[t];
                    bi = amn[t];
                }
            amv[blockIdx.x] = bv;
            ami[blockIdx.x] = bi;
        }
        return;
    }
    if (ks == 0 && g == 0 && live) store_y<YT>(y + o, GU ? silu_mul(acc[0], acc[R - 1]) : acc[0]);
}

// ------------------------------------------------------------------ generic exact kernel
// One wave per output (row, or gate/up row pair); lanes stride over 32-weight
// sub-blocks, dequantize them exactly to f32 and dot with up to 8
// activation rows read with scalar loads (any alignment).
template <int QT, bool GU, typename XT, typename YT>
__global__ __launch_bounds__(256) void k_gemv_generic(const uint8_t* __restrict__ Wq, const uint8_t* __restrict__ Wa,
                                                     const XT* __restrict__ x, YT* __restrict__ y, int M,
                                                     int64_t nout, int K, int64_t up_off, int64_t ldy,
                                                     int64_t nrows) {
    const int lane = threadIdx.x & 63;
    const int64_t o = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (o >= nout) return;
    constexpr int NR = GU ? 2 : 1;
    float acc[NR][8];
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int m = 0; m < 8; ++m) acc[r][m] = 0.0f;
    const int nsub = K >> 5;
    for (int sbi = lane; sbi < nsub; sbi += 64) {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const int64_t row = o + (r ? up_off : 0);
            float wv[32];
            if (QT == 14) {
                // Q6_K: sub-block sbi is half o of 64-weight step g = sbi / 2
                // (thq_dev.hpp, q6k_layout)
                const Q6Layout L = q6k_layout(nrows, K);
                const int g = sbi >> 1, o = sbi & 1;
                const uint8_t* ql = Wq + row * (K / 2) + g * 32;
                const uint8_t* qh = Wq + L.qh + row * (K / 4) + g * 16;
                const int8_t* sc = reinterpret_cast<const int8_t*>(Wq + L.sc + row * (K / 16) + g * 4 + 2 * o);
                const float d = f16_to_f32(reinterpret_cast<const uint16_t*>(Wq + L.d)[row * (K / 256) + (g >> 2)]);
                const float ds0 = d * (float)sc[0], ds1 = d * (float)sc[1];
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    const int code = ((ql[i] >> (4 * o)) & 0xF) | (((qh[i & 15] >> (2 * (2 * o + (i >> 4)))) & 3) << 4);
                    wv[i] = (i < 16 ? ds0 : ds1) * (float)(code - 32);  // (d * sc) * q, candle's order
                }
            } else if (QT != 8) {
                // affine weights may pad K to whole superblocks: address with the padded count
                const int nsb = (K + 255) >> 8, s = sbi >> 3, j = sbi & 7;
                uint4 h;
                h.x = *reinterpret_cast<const uint32_t*>(Wq + q4k_hdword(row, nsb, s, 0));
                h.y = *reinterpret_cast<const uint32_t*>(Wq + q4k_hdword(row, nsb, s, 1));
                h.z = *reinterpret_cast<const uint32_t*>(Wq + q4k_hdword(row, nsb, s, 2));
                h.w = *reinterpret_cast<const uint32_t*>(Wq + q4k_hdword(row, nsb, s, 3));
                float d1, m1;
                if (QT == 13) {
                    const uint32_t hw = (j >> 1) == 0 ? h.x : ((j >> 1) == 1 ? h.y : ((j >> 1) == 2 ? h.z : h.w));
                    d1 = aff_scale(hw);
                    m1 = -aff_bias(hw);  // w = scale * q - (-bias)
                } else {
                    uint32_t sc, mm;
                    q4k_hdr_sm(h, j, sc, mm);
                    d1 = q4k_hdr_d(h) * (float)sc;
                    m1 = q4k_hdr_dmin(h) * (float)mm;
                }
                const int sh = (j & 1) * 4;
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const uint8_t* q = Wq + q4k_piece(row, nsb, s, hh, j >> 1);
#pragma unroll
                    for (int i = 0; i < 16; ++i) wv[16 * hh + i] = d1 * (float)((q[i] >> sh) & 0xF) - m1;
                }
            } else {
                const int8_t* q0 = reinterpret_cast<const int8_t*>(Wq) + q8t_q(row, nsub, sbi, 0);
                const int8_t* q1 = reinterpret_cast<const int8_t*>(Wq) + q8t_q(row, nsub, sbi, 1);
                const float d = f16_to_f32(reinterpret_cast<const uint16_t*>(Wa)[q8t_d(row, nsub, sbi)]);
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    wv[i] = (float)q0[i] * d;
                    wv[16 + i] = (float)q1[i] * d;
                }
            }
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                if (m < M) {
                    const XT* xr = x + (int64_t)m * K + 32 * sbi;
                    float s = 0.0f;
#pragma unroll
                    for (int i = 0; i < 32; ++i) s = __builtin_fmaf(load_x<XT>(xr + i), wv[i], s);
                    acc[r][m] += s;
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        if (m >= M) break;
        const float g = wave_sum(acc[0][m]);
        const float u = GU ? wave_sum(acc[NR - 1][m]) : 0.0f;
        if (lane == 0) store_y<YT>(y + (int64_t)m * ldy + o, GU ? silu_mul(g, u) : g);
    }
}

// ------------------------------------------------------------------ launchers
static inline int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

// resident waves per CU (tunable: THQ_GEMV_WPC)
template <bool GU, bool AFF, typename YT>
static void launch_q4k_bf16_t(const uint8_t* W, const bf16_t* x, YT* y, int64_t nout, int K, int64_t up_off,
                              hipStream_t s, AmaxOut* am) {
    const int64_t nquads = (nout + 3) / 4;
    const int wpc = env_int("THQ_GEMV_WPC", 8);
    int64_t waves = (int64_t)256 * (wpc > 0 ? wpc : 8);
    if (waves > nquads) waves = nquads;
    const size_t lds = (size_t)K * 2;
    if (K <= 4096 && env_int("THQ_GEMV_ONESHOT", 1)) {
        float* amv = nullptr;
        uint32_t* ami = nullptr;
        if (am) {  // one partial per row quad (M = 1)
            if (GU || nquads > am->ld) return;
            amv = am->v;
            ami = am->i;
            am->nb = nquads;
        }
        if (K == 4096)
            hipLaunchKernelGGL((k_gemv1_q4k_bf16_1s<GU, AFF, true, YT>), dim3((unsigned)((nquads + 3) / 4)), dim3(256),
                               lds, s, W, x, y, nout, K, up_off, nquads, amv, ami);
        else
            hipLaunchKernelGGL((k_gemv1_q4k_bf16_1s<GU, AFF, false, YT>), dim3((unsigned)((nquads + 3) / 4)), dim3(256),
                               lds, s, W, x, y, nout, K, up_off, nquads, amv, ami);
        return;
    }
    if (am) return;  // no fused epilogue on the K-split / persistent kernels
    if (K <= 4 * 4096 && env_int("THQ_GEMV_ONESHOT", 1)) {
        // 2 quads per block (twice the blocks of 4) measured 8.4 -> 8.25 us at K = 12288
        static const int qpb = env_int("THQ_GEMV_QPB", 2) == 4 ? 4 : 2;
        const dim3 grid((unsigned)((nquads + qpb - 1) / qpb));
#define THQ_KS(KC_, QPB_) \
    hipLaunchKernelGGL((k_gemv1_q4k_bf16_ks<KC_, QPB_, GU, AFF, YT>), grid, dim3(64 * QPB_ * KC_), lds, s, W, x, y, nout, K, up_off, nquads)
        const int kc = (K + 4095) / 4096;
        if (qpb == 2) {
            if (kc == 2) THQ_KS(2, 2); else if (kc == 3) THQ_KS(3, 2); else THQ_KS(4, 2);
        } else {
            if (kc == 2) THQ_KS(2, 4); else if (kc == 3) THQ_KS(3, 4); else THQ_KS(4, 4);
        }
#undef THQ_KS
        return;
    }
    const unsigned grid = (unsigned)((waves + 3) / 4);
    switch ((K / 256 + 15) / 16) {
        case 1: hipLaunchKernelGGL((k_gemv1_q4k_bf16<1, GU, AFF, YT>), dim3(grid), dim3(256), lds, s, W, x, y, nout, K, up_off, nquads); break;
        case 2: hipLaunchKernelGGL((k_gemv1_q4k_bf16<2, GU, AFF, YT>), dim3(grid), dim3(256), lds, s, W, x, y, nout, K, up_off, nquads); break;
        case 3: hipLaunchKernelGGL((k_gemv1_q4k_bf16<3, GU, AFF, YT>), dim3(grid), dim3(256), lds, s, W, x, y, nout, K, up_off, nquads); break;
        default: hipLaunchKernelGGL((k_gemv1_q4k_bf16<4, GU, AFF, YT>), dim3(grid), dim3(256), lds, s, W, x, y, nout, K, up_off, nquads); break;
    }
}

template <bool GU, bool AFF, typename YT>
static hipError_t gemv1_q4k_t(const uint8_t* W, const void* x, bool xf32, YT* y, int64_t nout, int K, int64_t up_off,
                              hipStream_t s, AmaxOut* am) {
    const int kc = (K + 4095) / 4096;
    if (!xf32) {
        launch_q4k_bf16_t<GU, AFF, YT>(W, static_cast<const bf16_t*>(x), y, nout, K, up_off, s, am);
    } else if (am) {
        return hipSuccess;  // no fused epilogue on the f32-x kernel
    } else {
        const float* xf = static_cast<const float*>(x);
        constexpr int RR = GU ? 2 : 1;
        const unsigned grid = (unsigned)((nout + 3) / 4);
#define THQ_F32(KC_) \
    hipLaunchKernelGGL((k_gemv1_q4k_f32<KC_, RR, GU, AFF, YT>), dim3(grid), dim3(256), 0, s, W, xf, y, nout, K, up_off)
        switch (kc) {
            case 1: THQ_F32(1); break;
            case 2: THQ_F32(2); break;
            case 3: THQ_F32(3); break;
            case 4: THQ_F32(4); break;
            default: return hipErrorInvalidValue;
        }
#undef THQ_F32
    }
    return hipGetLastError();
}

// K ranges per tile: enough waves for the GPU (LM head: 4748 tiles, one
// range; 12288 rows: 384 tiles, four ranges)
template <bool GU, typename XT, typename YT>
static void launch_q8_t(const int8_t* Q, const uint16_t* D, const XT* x, YT* y, int64_t nout, int K, int64_t up_off,
                        hipStream_t s, AmaxOut* am) {
    const int64_t tiles = (nout + 31) / 32;
    const int nch = (K / 32 + 7) / 8;
    const int ks = (tiles >= 2048 || nch < 2) ? 1 : ((tiles >= 1024 || nch < 4) ? 2 : 4);
    const int tpb = 4 / ks;
    const int64_t blocks = (tiles + tpb - 1) / tpb;
    float* amv = nullptr;
    uint32_t* ami = nullptr;
    if (am) {  // one partial per block (M = 1)
        if (GU || blocks > am->ld) return;
        amv = am->v;
        ami = am->i;
        am->nb = blocks;
    }
#define THQ_Q8T(KS_)                                                                                            \
    do {                                                                                                        \
        if (K % 256 == 0)                                                                                       \
            hipLaunchKernelGGL((k_gemv1_q8<KS_, true, GU, XT, YT>), dim3((unsigned)blocks), dim3(256), 0, s, Q, D, \
                               x, y, nout, K, up_off, amv, ami);                                                \
        else                                                                                                    \
            hipLaunchKernelGGL((k_gemv1_q8<KS_, false, GU, XT, YT>), dim3((unsigned)blocks), dim3(256), 0, s, Q,   \
                               D, x, y, nout, K, up_off, amv, ami);                                             \
    } while (0)
    if (ks == 1) THQ_Q8T(1);
    else if (ks == 2) THQ_Q8T(2);
    else THQ_Q8T(4);
#undef THQ_Q8T
}

template <bool GU, typename XT, typename YT>
static hipError_t gemv1_q8_t(const int8_t* Q, const uint16_t* D, const XT* x, YT* y, int64_t nout, int K,
                             int64_t up_off, hipStream_t s, AmaxOut* am) {
    if (K > Q8T_KMAX || K % 32) return hipErrorInvalidValue;
    launch_q8_t<GU, XT, YT>(Q, D, x, y, nout, K, up_off, s, am);
    return hipGetLastError();
}

bool gemv_rows_supported(int qtype, int M, int K, bool gu, int64_t n_rows) {
    return (qtype == 12 || qtype == 13) && M >= 2 && M <= (K <= 4096 ? 4 : 2) && K % 256 == 0 &&
           K <= 4 * 4096 && (!gu || (n_rows / 2) % 4 == 0);
}

template <int MR, bool GU, bool AFF, typename YT>
static void rows_t(const uint8_t* W, const bf16_t* x, YT* y, int M, int64_t nout, int K, int64_t up_off,
                   hipStream_t s) {
    const int64_t nquads = (nout + 3) / 4;
    const dim3 grid((unsigned)((nquads + 3) / 4));
    const size_t lds = (size_t)MR * K * 2;
    if (K == 4096)
        hipLaunchKernelGGL((k_gemv_q4k_bf16_rows<MR, GU, AFF, true, YT>), grid, dim3(256), lds, s, W, x, y, M, nout, K,
                           up_off, nquads);
    else
        hipLaunchKernelGGL((k_gemv_q4k_bf16_rows<MR, GU, AFF, false, YT>), grid, dim3(256), lds, s, W, x, y, M, nout,
                           K, up_off, nquads);
}

template <bool GU, bool AFF, typename YT>
static hipError_t rows_m(const uint8_t* W, const bf16_t* x, YT* y, int M, int64_t nout, int K, int64_t up_off,
                         hipStream_t s) {
    if (K > 4096) {  // two rows, K split over KC waves per row-quad pair
        const int64_t nquads = (nout + 3) / 4;
        const dim3 grid((unsigned)((nquads + 1) / 2));
        const size_t lds = (size_t)2 * K * 2;
#define THQ_KSR(KC_) \
    hipLaunchKernelGGL((k_gemv_q4k_bf16_ks_rows<KC_, GU, AFF, YT>), grid, dim3(128 * KC_), lds, s, W, x, y, M, nout, K, up_off, nquads)
        const int kc = (K + 4095) / 4096;
        if (kc == 2) THQ_KSR(2); else if (kc == 3) THQ_KSR(3); else THQ_KSR(4);
#undef THQ_KSR
        return hipGetLastError();
    }
    if (M == 2) rows_t<2, GU, AFF, YT>(W, x, y, M, nout, K, up_off, s);
    else rows_t<4, GU, AFF, YT>(W, x, y, M, nout, K, up_off, s);
    return hipGetLastError();
}

hipError_t launch_gemv_rows(const WeightView& w, const void* x, void* y, bool yf32, bool gu, int M, int64_t nout,
                            int64_t up_off, hipStream_t s) {
    const int K = (int)w.K;
    if (!gemv_rows_supported(w.qtype, M, K, gu, w.N)) return hipErrorInvalidValue;
    const bf16_t* xb = static_cast<const bf16_t*>(x);
#define THQ_R(GU_, AFF_)                                                                   \
    (yf32 ? rows_m<GU_, AFF_, float>(w.q, xb, (float*)y, M, nout, K, up_off, s)             \
          : rows_m<GU_, AFF_, bf16_t>(w.q, xb, (bf16_t*)y, M, nout, K, up_off, s))
    if (w.qtype == 13) return gu ? THQ_R(true, true) : THQ_R(false, true);
    return gu ? THQ_R(true, false) : THQ_R(false, false);
#undef THQ_R
}

bool gemv1_supported(int qtype, int K, bool gu, int64_t n_rows) {
    if (qtype == 14) return K % 256 == 0 && K <= 4 * 4096;
    if (qtype != 8) return K % 256 == 0 && K <= 4 * 4096 && (!gu || (n_rows / 2) % 4 == 0);
    return K % 32 == 0 && K <= 8 * 1024;
}

hipError_t launch_gemv1(const WeightView& w, const void* x, bool xf32, void* y, bool yf32, bool gu, int64_t nout,
                        int64_t up_off, hipStream_t s, AmaxOut* am) {
    const int K = (int)w.K;
    if (w.qtype == 14) {
        if (xf32) return am ? hipSuccess : launch_generic(w, x, xf32, y, yf32, gu, 1, nout, up_off, s);
        return launch_gemv1_q6k(w, x, y, yf32, gu, nout, up_off, s, am);
    }
    if (w.qtype == 12) {
        if (gu) {
            return yf32 ? gemv1_q4k_t<true, false, float>(w.q, x, xf32, (float*)y, nout, K, up_off, s, am)
                        : gemv1_q4k_t<true, false, bf16_t>(w.q, x, xf32, (bf16_t*)y, nout, K, up_off, s, am);
        }
        return yf32 ? gemv1_q4k_t<false, false, float>(w.q, x, xf32, (float*)y, nout, K, up_off, s, am)
                    : gemv1_q4k_t<false, false, bf16_t>(w.q, x, xf32, (bf16_t*)y, nout, K, up_off, s, am);
    }
    if (w.qtype == 13) {
        if (gu) {
            return yf32 ? gemv1_q4k_t<true, true, float>(w.q, x, xf32, (float*)y, nout, K, up_off, s, am)
                        : gemv1_q4k_t<true, true, bf16_t>(w.q, x, xf32, (bf16_t*)y, nout, K, up_off, s, am);
        }
        return yf32 ? gemv1_q4k_t<false, true, float>(w.q, x, xf32, (float*)y, nout, K, up_off, s, am)
                    : gemv1_q4k_t<false, true, bf16_t>(w.q, x, xf32, (bf16_t*)y, nout, K, up_off, s, am);
    }
    const int8_t* Q = reinterpret_cast<const int8_t*>(w.q);
    const uint16_t* D = reinterpret_cast<const uint16_t*>(w.aux);
#define THQ_Q8(GU_, XT_, YT_) gemv1_q8_t<GU_, XT_, YT_>(Q, D, (const XT_*)x, (YT_*)y, nout, K, up_off, s, am)
    if (gu) {
        if (xf32) return yf32 ? THQ_Q8(true, float, float) : THQ_Q8(true, float, bf16_t);
        return yf32 ? THQ_Q8(true, bf16_t, float) : THQ_Q8(true, bf16_t, bf16_t);
    }
    if (xf32) return yf32 ? THQ_Q8(false, float, float) : THQ_Q8(false, float, bf16_t);
    return yf32 ? THQ_Q8(false, bf16_t, float) : THQ_Q8(false, bf16_t, bf16_t);
#undef THQ_Q8
}

template <int QT, bool GU, typename XT, typename YT>
static hipError_t generic_t(const WeightView& w, const XT* x, YT* y, int M, int64_t nout, int64_t up_off,
                            int64_t ldy, hipStream_t s) {
    for (int m0 = 0; m0 < M; m0 += 8) {
        const int mm = M - m0 < 8 ? M - m0 : 8;
        hipLaunchKernelGGL((k_gemv_generic<QT, GU, XT, YT>), dim3((unsigned)((nout + 3) / 4)), dim3(256), 0, s, w.q,
                           w.aux, x + (int64_t)m0 * w.K, y + (int64_t)m0 * ldy, mm, nout, (int)w.K, up_off, ldy, w.N);
    }
    return hipGetLastError();
}

hipError_t launch_generic(const WeightView& w, const void* x, bool xf32, void* y, bool yf32, bool gu, int M,
                          int64_t nout, int64_t up_off, hipStream_t s) {
    const int64_t ldy = nout;
#define THQ_G(QT_, GU_, XT_, YT_) generic_t<QT_, GU_, XT_, YT_>(w, (const XT_*)x, (YT_*)y, M, nout, up_off, ldy, s)
#define THQ_G2(QT_, GU_)                                                              \
    (xf32 ? (yf32 ? THQ_G(QT_, GU_, float, float) : THQ_G(QT_, GU_, float, bf16_t))   \
          : (yf32 ? THQ_G(QT_, GU_, bf16_t, float) : THQ_G(QT_, GU_, bf16_t, bf16_t)))
    if (w.qtype == 12) return gu ? THQ_G2(12, true) : THQ_G2(12, false);
    if (w.qtype == 13) return gu ? THQ_G2(13, true) : THQ_G2(13, false);
    if (w.qtype == 14) return gu ? THQ_G2(14, true) : THQ_G2(14, false);
    return gu ? THQ_G2(8, true) : THQ_G2(8, false);
#undef THQ_G2
#undef THQ_G
}

}  // namespace thq
