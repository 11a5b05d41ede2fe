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

namespace thq {

// ------------------------------------------------------------------ helpers
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    bf16x2_t av, bv;
    __builtin_memcpy(&av, &a, 4);
    __builtin_memcpy(&bv, &b, 4);
    return __builtin_amdgcn_fdot2_f32_bf16(av, bv, c, false);
}

// row index of slot r for a wave that starts at row0; in gate/up mode the
// wave owns outputs i0 .. i0+R/2-1 and its slots alternate gate/up rows
template <int R, bool GU>
__device__ __forceinline__ int64_t slot_row(int64_t base, int r, int64_t up_off) {
    if (GU) return base + (r >> 1) + ((r & 1) ? up_off : 0);
    return base + r;
}

template <int R, bool GU, typename YT>
__device__ __forceinline__ void write_rows(YT* __restrict__ y, int64_t base, int64_t nout, const float* acc) {
    if (threadIdx.x % 64 != 0) return;
    if (GU) {
#pragma unroll
        for (int p = 0; p < R / 2; ++p)
            if (base + p < nout) store_y<YT>(y + base + p, silu_mul(acc[2 * p], acc[2 * p + 1]));
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (base + r < nout) store_y<YT>(y + base + r, acc[r]);
    }
}

// ------------------------------------------------------------------ Q4_K M=1, bf16 x
// KC = number of 4096-wide K chunks (K <= 4096*KC).  R rows per wave.
template <int KC, int R, bool GU, typename YT>
__global__ __launch_bounds__(256) void k_gemv1_q4k_bf16(const uint8_t* __restrict__ W, const bf16_t* __restrict__ x,
                                                       YT* __restrict__ y, int64_t nout, int K, int64_t up_off) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t base = wave * (GU ? R / 2 : R);
    if (base >= nout) return;
    const int nsb = K >> 8;
    const int64_t rb = (int64_t)nsb * THQ_Q4K_BYTES;
    const int sl = lane >> 2, part = lane & 3;

    // activations for this lane: pairs (x[2i], x[2i+1]) of both sub-blocks
    uint32_t xlo[KC][16], xhi[KC][16];
    float sxlo[KC], sxhi[KC];
#pragma unroll
    for (int c = 0; c < KC; ++c) {
        const int s = 16 * c + sl;
        sxlo[c] = 0.0f;
        sxhi[c] = 0.0f;
        if (s < nsb) {
            const uint4* xp = reinterpret_cast<const uint4*>(x + (int64_t)s * 256 + 64 * part);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint4 a = xp[v], b = xp[4 + v];
                xlo[c][4 * v] = a.x; xlo[c][4 * v + 1] = a.y; xlo[c][4 * v + 2] = a.z; xlo[c][4 * v + 3] = a.w;
                xhi[c][4 * v] = b.x; xhi[c][4 * v + 1] = b.y; xhi[c][4 * v + 2] = b.z; xhi[c][4 * v + 3] = b.w;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                sxlo[c] += bf16_to_f32(xlo[c][i] & 0xFFFF) + bf16_to_f32(xlo[c][i] >> 16);
                sxhi[c] += bf16_to_f32(xhi[c][i] & 0xFFFF) + bf16_to_f32(xhi[c][i] >> 16);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) { xlo[c][i] = 0; xhi[c][i] = 0; }
        }
    }

    // issue every weight load of the wave before any math
    uint4 hdr[R][KC], q0[R][KC], q1[R][KC];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        int64_t row = slot_row<R, GU>(base, r, up_off);
        const bool ok = GU ? (base + (r >> 1) < nout) : (row < nout);
        if (!ok) row = GU ? up_off * (r & 1) : 0;
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const int s = 16 * c + sl;
            if (s < nsb) {
                const uint8_t* blk = W + row * rb + (int64_t)s * THQ_Q4K_BYTES;
                hdr[r][c] = *reinterpret_cast<const uint4*>(blk);
                q0[r][c] = *reinterpret_cast<const uint4*>(blk + 16 + 32 * part);
                q1[r][c] = *reinterpret_cast<const uint4*>(blk + 32 + 32 * part);
            } else {
                hdr[r][c] = make_uint4(0, 0, 0, 0);
                q0[r][c] = hdr[r][c];
                q1[r][c] = hdr[r][c];
            }
        }
    }

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float a = 0.0f;
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const uint32_t qw[8] = {q0[r][c].x, q0[r][c].y, q0[r][c].z, q0[r][c].w,
                                    q1[r][c].x, q1[r][c].y, q1[r][c].z, q1[r][c].w};
            float alo = 0.0f, ahi = 0.0f;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const uint32_t p0 = __builtin_amdgcn_perm(0u, qw[t], 0x0c010c00u);  // bytes 4t, 4t+1
                const uint32_t p1 = __builtin_amdgcn_perm(0u, qw[t], 0x0c030c02u);  // bytes 4t+2, 4t+3
                // (q | 0x4300) is the bf16 of 128 + q
                alo = dot2_bf16((p0 & 0x000F000Fu) | 0x43004300u, xlo[c][2 * t], alo);
                alo = dot2_bf16((p1 & 0x000F000Fu) | 0x43004300u, xlo[c][2 * t + 1], alo);
                ahi = dot2_bf16(((p0 >> 4) & 0x000F000Fu) | 0x43004300u, xhi[c][2 * t], ahi);
                ahi = dot2_bf16(((p1 >> 4) & 0x000F000Fu) | 0x43004300u, xhi[c][2 * t + 1], ahi);
            }
            const float dlo = alo - 128.0f * sxlo[c];  // sum x*q over sub-block 2p
            const float dhi = ahi - 128.0f * sxhi[c];  // sum x*q over sub-block 2p+1
            const uint4 h = hdr[r][c];
            uint32_t sc0, m0, sc1, m1;
            scale_min_k4(2 * part, h.y, h.z, h.w, sc0, m0);
            scale_min_k4(2 * part + 1, h.y, h.z, h.w, sc1, m1);
            const float d = f16_to_f32(h.x & 0xFFFF), dmin = f16_to_f32(h.x >> 16);
            a = __builtin_fmaf(d, (float)sc0 * dlo + (float)sc1 * dhi, a);
            a = __builtin_fmaf(-dmin, (float)m0 * sxlo[c] + (float)m1 * sxhi[c], a);
        }
        acc[r] = wave_sum(a);
    }
    write_rows<R, GU, YT>(y, base, nout, acc);
}

// ------------------------------------------------------------------ Q4_K M=1, f32 x
template <int KC, int R, bool GU, typename YT>
__global__ __launch_bounds__(256) void k_gemv1_q4k_f32(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                      YT* __restrict__ y, int64_t nout, int K, int64_t up_off) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t base = wave * (GU ? R / 2 : R);
    if (base >= nout) return;
    const int nsb = K >> 8;
    const int64_t rb = (int64_t)nsb * THQ_Q4K_BYTES;
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
            const uint8_t* blk = W + row * rb + (int64_t)s * THQ_Q4K_BYTES;
            const uint4 h = *reinterpret_cast<const uint4*>(blk);
            const uint4 a4 = *reinterpret_cast<const uint4*>(blk + 16 + 32 * part);
            const uint4 b4 = *reinterpret_cast<const uint4*>(blk + 32 + 32 * part);
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
            uint32_t sc0, m0, sc1, m1;
            scale_min_k4(2 * part, h.y, h.z, h.w, sc0, m0);
            scale_min_k4(2 * part + 1, h.y, h.z, h.w, sc1, m1);
            const float d = f16_to_f32(h.x & 0xFFFF), dmin = f16_to_f32(h.x >> 16);
            acc[r] = __builtin_fmaf(d, (float)sc0 * dl + (float)sc1 * dh, acc[r]);
            acc[r] = __builtin_fmaf(-dmin, (float)m0 * sxl + (float)m1 * sxh, acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
    write_rows<R, GU, YT>(y, base, nout, acc);
}

// ------------------------------------------------------------------ Q8_0 M=1
// Planes: qs [N][K] i8, d [N][K/32] f16.  Lane l covers 16 bytes of every
// 1024-wide K chunk: k = 1024c + 16l (block 32c + l/2).  u = q ^ 0x80 is the
// unsigned byte q + 128, converted with v_cvt_f32_ubyte; the 128 offset is
// removed with the lane's sum of x.
template <int KC, int R, bool GU, typename XT, typename YT>
__global__ __launch_bounds__(256) void k_gemv1_q8(const int8_t* __restrict__ Q, const uint16_t* __restrict__ D,
                                                 const XT* __restrict__ x, YT* __restrict__ y, int64_t nout, int K,
                                                 int64_t up_off) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t base = wave * (GU ? R / 2 : R);
    if (base >= nout) return;
    const int nb = K >> 5;

    float xv[KC][16], sx[KC];
#pragma unroll
    for (int c = 0; c < KC; ++c) {
        const int k0 = 1024 * c + 16 * lane;
        sx[c] = 0.0f;
        if (k0 < K) {
#pragma unroll
            for (int i = 0; i < 16; ++i) xv[c][i] = load_x<XT>(x + k0 + i);
#pragma unroll
            for (int i = 0; i < 16; ++i) sx[c] += xv[c][i];
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) xv[c][i] = 0.0f;
        }
    }
    uint4 qv[R][KC];
    uint16_t dv[R][KC];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        int64_t row = slot_row<R, GU>(base, r, up_off);
        const bool ok = GU ? (base + (r >> 1) < nout) : (row < nout);
        if (!ok) row = GU ? up_off * (r & 1) : 0;
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const int k0 = 1024 * c + 16 * lane;
            if (k0 < K) {
                qv[r][c] = *reinterpret_cast<const uint4*>(Q + row * K + k0);
                dv[r][c] = D[row * nb + (k0 >> 5)];
            } else {
                qv[r][c] = make_uint4(0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u);
                dv[r][c] = 0;
            }
        }
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float a = 0.0f;
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const uint32_t w4[4] = {qv[r][c].x ^ 0x80808080u, qv[r][c].y ^ 0x80808080u, qv[r][c].z ^ 0x80808080u,
                                    qv[r][c].w ^ 0x80808080u};
            float s = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                s = __builtin_fmaf(ubyte_f32<0>(w4[t]), xv[c][4 * t], s);
                s = __builtin_fmaf(ubyte_f32<1>(w4[t]), xv[c][4 * t + 1], s);
                s = __builtin_fmaf(ubyte_f32<2>(w4[t]), xv[c][4 * t + 2], s);
                s = __builtin_fmaf(ubyte_f32<3>(w4[t]), xv[c][4 * t + 3], s);
            }
            a = __builtin_fmaf(f16_to_f32(dv[r][c]), s - 128.0f * sx[c], a);
        }
        acc[r] = wave_sum(a);
    }
    write_rows<R, GU, YT>(y, base, nout, acc);
}

// ------------------------------------------------------------------ generic exact kernel
// One wave per output (row, or gate/up row pair); lanes stride over 32-weight
// sub-blocks, dequantize them exactly to f32 and dot with up to 8
// activation rows read with scalar loads (any alignment).
template <int QT, bool GU, typename XT, typename YT>
__global__ __launch_bounds__(256) void k_gemv_generic(const uint8_t* __restrict__ Wq, const uint16_t* __restrict__ Wd,
                                                     const XT* __restrict__ x, YT* __restrict__ y, int M,
                                                     int64_t nout, int K, int64_t up_off, int64_t ldy) {
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
            if (QT == 12) {
                const uint8_t* blk = Wq + row * (int64_t)(K >> 8) * THQ_Q4K_BYTES + (int64_t)(sbi >> 3) * THQ_Q4K_BYTES;
                const int j = sbi & 7;
                const uint4 h = *reinterpret_cast<const uint4*>(blk);
                uint32_t sc, mm;
                scale_min_k4(j, h.y, h.z, h.w, sc, mm);
                const float d1 = f16_to_f32(h.x & 0xFFFF) * (float)sc, m1 = f16_to_f32(h.x >> 16) * (float)mm;
                const uint8_t* q = blk + 16 + 32 * (j >> 1);
                const int sh = (j & 1) * 4;
#pragma unroll
                for (int i = 0; i < 32; ++i) wv[i] = d1 * (float)((q[i] >> sh) & 0xF) - m1;
            } else {
                const int8_t* q = reinterpret_cast<const int8_t*>(Wq) + row * K + 32 * sbi;
                const float d = f16_to_f32(Wd[row * nsub + sbi]);
#pragma unroll
                for (int i = 0; i < 32; ++i) wv[i] = (float)q[i] * d;
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

template <int KC, int R, bool GU, typename YT>
static void launch_q4k_bf16_t(const uint8_t* W, const bf16_t* x, YT* y, int64_t nout, int K, int64_t up_off,
                              hipStream_t s) {
    const int64_t per_wave = GU ? R / 2 : R;
    const int64_t waves = (nout + per_wave - 1) / per_wave;
    hipLaunchKernelGGL((k_gemv1_q4k_bf16<KC, R, GU, YT>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, W, x,
                       y, nout, K, up_off);
}

template <int KC, bool GU, typename YT>
static void pick_r_q4k_bf16(int R, const uint8_t* W, const bf16_t* x, YT* y, int64_t nout, int K, int64_t up_off,
                            hipStream_t s) {
    if constexpr (GU) {
        if (R >= 4) launch_q4k_bf16_t<KC, 4, GU, YT>(W, x, y, nout, K, up_off, s);
        else launch_q4k_bf16_t<KC, 2, GU, YT>(W, x, y, nout, K, up_off, s);
    } else {
        if (R >= 4) launch_q4k_bf16_t<KC, 4, GU, YT>(W, x, y, nout, K, up_off, s);
        else if (R == 2) launch_q4k_bf16_t<KC, 2, GU, YT>(W, x, y, nout, K, up_off, s);
        else launch_q4k_bf16_t<KC, 1, GU, YT>(W, x, y, nout, K, up_off, s);
    }
}

// default rows per wave: enough waves to fill 256 CUs several times over
static int default_r(int64_t nrows, int kc) {
    const int r = env_int("THQ_GEMV_R", 0);
    if (r > 0) return r;
    if (kc >= 2) return 1;
    return nrows >= 8192 ? 2 : 1;
}

template <bool GU, typename YT>
static hipError_t gemv1_q4k_t(const uint8_t* W, const void* x, bool xf32, YT* y, int64_t nout, int K,
                              int64_t up_off, hipStream_t s) {
    const int kc = (K + 4095) / 4096;
    const int R = default_r(GU ? 2 * nout : nout, kc) * (GU ? 2 : 1);
    if (!xf32) {
        const bf16_t* xb = static_cast<const bf16_t*>(x);
        switch (kc) {
            case 1: pick_r_q4k_bf16<1, GU, YT>(R, W, xb, y, nout, K, up_off, s); break;
            case 2: pick_r_q4k_bf16<2, GU, YT>(R, W, xb, y, nout, K, up_off, s); break;
            case 3: pick_r_q4k_bf16<3, GU, YT>(R, W, xb, y, nout, K, up_off, s); break;
            case 4: pick_r_q4k_bf16<4, GU, YT>(R, W, xb, y, nout, K, up_off, s); break;
            default: return hipErrorInvalidValue;
        }
    } else {
        const float* xf = static_cast<const float*>(x);
        constexpr int RR = GU ? 2 : 1;
        const int64_t waves = nout;
        const unsigned grid = (unsigned)((waves + 3) / 4);
        switch (kc) {
            case 1: hipLaunchKernelGGL((k_gemv1_q4k_f32<1, RR, GU, YT>), dim3(grid), dim3(256), 0, s, W, xf, y, nout, K, up_off); break;
            case 2: hipLaunchKernelGGL((k_gemv1_q4k_f32<2, RR, GU, YT>), dim3(grid), dim3(256), 0, s, W, xf, y, nout, K, up_off); break;
            case 3: hipLaunchKernelGGL((k_gemv1_q4k_f32<3, RR, GU, YT>), dim3(grid), dim3(256), 0, s, W, xf, y, nout, K, up_off); break;
            case 4: hipLaunchKernelGGL((k_gemv1_q4k_f32<4, RR, GU, YT>), dim3(grid), dim3(256), 0, s, W, xf, y, nout, K, up_off); break;
            default: return hipErrorInvalidValue;
        }
    }
    return hipGetLastError();
}

template <int KC, bool GU, typename XT, typename YT>
static void launch_q8_t(const int8_t* Q, const uint16_t* D, const XT* x, YT* y, int64_t nout, int K, int64_t up_off,
                        hipStream_t s) {
    constexpr int R = GU ? 2 : 1;
    const int64_t waves = nout;
    hipLaunchKernelGGL((k_gemv1_q8<KC, R, GU, XT, YT>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, Q, D, x, y,
                       nout, K, up_off);
}

template <bool GU, typename XT, typename YT>
static hipError_t gemv1_q8_t(const int8_t* Q, const uint16_t* D, const XT* x, YT* y, int64_t nout, int K,
                             int64_t up_off, hipStream_t s) {
    const int kc = (K + 1023) / 1024;
    switch (kc) {
        case 1: launch_q8_t<1, GU, XT, YT>(Q, D, x, y, nout, K, up_off, s); break;
        case 2: launch_q8_t<2, GU, XT, YT>(Q, D, x, y, nout, K, up_off, s); break;
        case 3: launch_q8_t<3, GU, XT, YT>(Q, D, x, y, nout, K, up_off, s); break;
        case 4: launch_q8_t<4, GU, XT, YT>(Q, D, x, y, nout, K, up_off, s); break;
        case 5: launch_q8_t<5, GU, XT, YT>(Q, D, x, y, nout, K, up_off, s); break;
        case 6: launch_q8_t<6, GU, XT, YT>(Q, D, x, y, nout, K, up_off, s); break;
        case 7: launch_q8_t<7, GU, XT, YT>(Q, D, x, y, nout, K, up_off, s); break;
        case 8: launch_q8_t<8, GU, XT, YT>(Q, D, x, y, nout, K, up_off, s); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool gemv1_supported(int qtype, int K) {
    if (qtype == 12) return K % 256 == 0 && K <= 4 * 4096;
    return K % 32 == 0 && K <= 8 * 1024;
}

hipError_t launch_gemv1(const WeightView& w, const void* x, bool xf32, void* y, bool yf32, bool gu, int64_t nout,
                        int64_t up_off, hipStream_t s) {
    const int K = (int)w.K;
    if (w.qtype == 12) {
        if (gu) {
            return yf32 ? gemv1_q4k_t<true, float>(w.q, x, xf32, (float*)y, nout, K, up_off, s)
                        : gemv1_q4k_t<true, bf16_t>(w.q, x, xf32, (bf16_t*)y, nout, K, up_off, s);
        }
        return yf32 ? gemv1_q4k_t<false, float>(w.q, x, xf32, (float*)y, nout, K, up_off, s)
                    : gemv1_q4k_t<false, bf16_t>(w.q, x, xf32, (bf16_t*)y, nout, K, up_off, s);
    }
    const int8_t* Q = reinterpret_cast<const int8_t*>(w.q);
#define THQ_Q8(GU_, XT_, YT_) gemv1_q8_t<GU_, XT_, YT_>(Q, w.d, (const XT_*)x, (YT_*)y, nout, K, up_off, s)
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
                           w.d, x + (int64_t)m0 * w.K, y + (int64_t)m0 * ldy, mm, nout, (int)w.K, up_off, ldy);
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
    return gu ? THQ_G2(8, true) : THQ_G2(8, false);
#undef THQ_G2
#undef THQ_G
}

}  // namespace thq
