// k_weights.hip — weight preparation kernels for gfx950:
//   * repack GGUF Q8_0 blocks (34 B, 2-byte aligned) into an aligned i8 plane
//     [N][K] plus an f16 scale plane [N][K/32]; GGUF Q4_K blocks into the
//     row-quad layout (thq_dev.hpp, q4k_group)
//   * quantize f32 weights on the device with candle's CPU rounding rules
//     ([ext] candle-core 0.11.0 k_quants.rs BlockQ8_0/BlockQ4K::from_float,
//     utils.rs make_qkx1_quants), bit-identical to the CPU quantizer
//   * exact f32 dequantization (BlockQ8_0/BlockQ4K::to_float)
//
// All f32 arithmetic here is compiled with -ffp-contract=off: each expression
// rounds exactly as written, like the Rust code it follows.
#include "thq_dev.hpp"
#include "thq_kernels.hpp"

namespace thq {

// ---------------------------------------------------------------- Q8_0 repack
__global__ __launch_bounds__(256) void k_repack_q8_0(const uint8_t* __restrict__ raw, int8_t* __restrict__ qs,
                                                     uint16_t* __restrict__ dpl, int64_t nblocks) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint16_t* src = reinterpret_cast<const uint16_t*>(raw + b * THQ_Q8_0_BYTES);  // 2-B aligned
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = (uint32_t)src[1 + 2 * i] | ((uint32_t)src[2 + 2 * i] << 16);
    dpl[b] = src[0];
    uint4* dst = reinterpret_cast<uint4*>(qs + b * THQ_QK8_0);
    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
}

// ---------------------------------------------------------------- quantize Q8_0
__device__ __forceinline__ int8_t sat_i8(float v) {
    if (v != v) return 0;
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    return (int8_t)v;
}

__global__ __launch_bounds__(256) void k_quantize_q8_0(const float* __restrict__ w, int8_t* __restrict__ qs,
                                                       uint16_t* __restrict__ dpl, int64_t nblocks) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float4* src = reinterpret_cast<const float4*>(w + b * THQ_QK8_0);
    float x[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float4 v = src[i];
        x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    _Float16 dh = (_Float16)d;
    uint16_t dbits;
    __builtin_memcpy(&dbits, &dh, 2);
    dpl[b] = dbits;
    uint32_t packed[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t v = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) v |= ((uint32_t)(uint8_t)sat_i8(roundf(x[4 * i + j] * id))) << (8 * j);
        packed[i] = v;
    }
    uint4* dst = reinterpret_cast<uint4*>(qs + b * THQ_QK8_0);
    dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
}

// ---------------------------------------------------------------- quantize Q4_K
__device__ __forceinline__ int nearest_int(float v) {
    const float r = roundf(v);  // half away from zero, like Rust's f32::round
    if (r != r) return 0;
    if (r >= 2147483647.0f) return 2147483647;
    if (r <= -2147483648.0f) return (-2147483647 - 1);
    return (int)r;
}

// make_qkx1_quants(15, 5, x[32]) -> (scale, -min); candle's utils.rs order.
__device__ void make_qkx1_quants_32(const float* x, float& scale_out, float& min_out) {
    float mn = x[0], mx = x[0];
#pragma unroll
    for (int i = 1; i < 32; ++i) {
        mn = x[i] < mn ? x[i] : mn;
        mx = x[i] > mx ? x[i] : mx;
    }
    if (mx == mn) {
        scale_out = 0.0f;
        min_out = 0.0f;
        return;
    }
    float min = mn < 0.0f ? mn : 0.0f;
    float iscale = 15.0f / (mx - min);
    float scale = 1.0f / iscale;
    uint8_t l[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) l[i] = 0;
    for (int it = 0; it < 5; ++it) {
        float sumlx = 0.0f;
        int suml2 = 0;
        bool did_change = false;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            int li = nearest_int(iscale * (x[i] - min));
            li = li < 0 ? 0 : (li > 15 ? 15 : li);
            if ((uint8_t)li != l[i]) {
                l[i] = (uint8_t)li;
                did_change = true;
            }
            sumlx += (x[i] - min) * (float)li;
            suml2 += li * li;
        }
        scale = sumlx / (float)suml2;
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) sum += x[i] - scale * (float)l[i];
        min = sum / 32.0f;
        if (min > 0.0f) min = 0.0f;
        iscale = 1.0f / scale;
        if (!did_change) break;
    }
    scale_out = scale;
    min_out = -min;
}

// 8 lanes per superblock: lane j runs make_qkx1_quants on sub-block j, the
// group OR-reduces the 6-bit scales into the on-device header (lanes 0..3
// write its four dwords), every lane requantizes its sub-block and the even
// lane of each pair writes the 32 shared nibble bytes as two 16-B pieces.
__global__ __launch_bounds__(256) void k_quantize_q4k(const float* __restrict__ w, uint8_t* __restrict__ dst,
                                                      int64_t nsuper, int nsb) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t sb = t >> 3;
    const int j = (int)(t & 7);
    const bool live = sb < nsuper;
    float x[32];
    const float4* src = reinterpret_cast<const float4*>(w + (live ? sb : 0) * THQ_QK_K + 32 * j);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float4 v = src[i];
        x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
    }
    float scale, minv;
    make_qkx1_quants_32(x, scale, minv);
    // group of 8 lanes: max scale, max min
    float max_scale = fmaxf(0.0f, scale), max_min = fmaxf(0.0f, minv);
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) {
        max_scale = fmaxf(max_scale, __shfl_xor(max_scale, off, 64));
        max_min = fmaxf(max_min, __shfl_xor(max_min, off, 64));
    }
    const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    const int lsi = nearest_int(inv_scale * scale);
    const int lmi = nearest_int(inv_min * minv);
    const uint32_t ls = (uint32_t)(uint8_t)(lsi < 63 ? lsi : 63);
    const uint32_t lm = (uint32_t)(uint8_t)(lmi < 63 ? lmi : 63);
    // on-device header: lane j owns 12 bits of H[j/2]; OR-reduce over the group
    uint32_t h0 = 0, h1 = 0, h2 = 0, h3 = 0;
    {
        const uint32_t f = (ls | (lm << 6)) << (12 * (j & 1));
        h0 = (j >> 1) == 0 ? f : 0u;
        h1 = (j >> 1) == 1 ? f : 0u;
        h2 = (j >> 1) == 2 ? f : 0u;
        h3 = (j >> 1) == 3 ? f : 0u;
    }
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) {
        h0 |= __shfl_xor(h0, off, 64);
        h1 |= __shfl_xor(h1, off, 64);
        h2 |= __shfl_xor(h2, off, 64);
        h3 |= __shfl_xor(h3, off, 64);
    }
    const _Float16 dh = (_Float16)(max_scale / 63.0f);
    const _Float16 mh = (_Float16)(max_min / 63.0f);
    // requantize this sub-block against the stored scale/min (ls, lm are what
    // get_scale_min_k4 returns for this sub-block: the packing is lossless)
    const float d = (float)dh * (float)ls;
    uint32_t L[8];  // 32 nibble values, one per byte
#pragma unroll
    for (int i = 0; i < 8; ++i) L[i] = 0;
    if (d != 0.0f) {
        const float dm = (float)mh * (float)lm;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            int lv = nearest_int((x[i] + dm) / d);
            lv = lv < 0 ? 0 : (lv > 15 ? 15 : lv);
            L[i >> 2] |= (uint32_t)lv << (8 * (i & 3));
        }
    }
    // odd sub-block supplies the high nibbles of the even one's bytes
    uint32_t P[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t other = __shfl_xor(L[i], 1, 64);
        P[i] = (j & 1) ? 0u : (L[i] | (other << 4));
    }
    if (!live) return;
    const int64_t n = sb / nsb;
    const int sidx = (int)(sb - n * nsb);
    if (j < 4) {  // header dword j of this row
        uint16_t dbits, mbits;
        __builtin_memcpy(&dbits, &dh, 2);
        __builtin_memcpy(&mbits, &mh, 2);
        const uint32_t dd = (uint32_t)dbits | ((uint32_t)mbits << 16);
        const uint32_t hw = j == 0 ? h0 : (j == 1 ? h1 : (j == 2 ? h2 : h3));
        *reinterpret_cast<uint32_t*>(dst + q4k_hdword(n, nsb, sidx, j)) = hw | (((dd >> (8 * j)) & 0xFFu) << 24);
    }
    if ((j & 1) == 0) {
        const int part = j >> 1;
        *reinterpret_cast<uint4*>(dst + q4k_piece(n, nsb, sidx, 0, part)) = make_uint4(P[0], P[1], P[2], P[3]);
        *reinterpret_cast<uint4*>(dst + q4k_piece(n, nsb, sidx, 1, part)) = make_uint4(P[4], P[5], P[6], P[7]);
    }
}

// ---------------------------------------------------------------- dequantize
// one thread per 32-weight block: y = q * d
__global__ __launch_bounds__(256) void k_dequant_q8_0(const int8_t* __restrict__ qs,
                                                      const uint16_t* __restrict__ dpl, float* __restrict__ out,
                                                      int64_t nblocks) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float d = f16_to_f32(dpl[b]);
    const uint4* src = reinterpret_cast<const uint4*>(qs + b * THQ_QK8_0);
    float4* dst = reinterpret_cast<float4*>(out + b * THQ_QK8_0);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint4 v = src[h];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float4 o;
            o.x = (float)(int8_t)(w[i] & 0xFF) * d;
            o.y = (float)(int8_t)((w[i] >> 8) & 0xFF) * d;
            o.z = (float)(int8_t)((w[i] >> 16) & 0xFF) * d;
            o.w = (float)(int8_t)(w[i] >> 24) * d;
            dst[4 * h + i] = o;
        }
    }
}

// one thread per (superblock, sub-block j): y = d*sc*q - dmin*m
__global__ __launch_bounds__(256) void k_dequant_q4k(const uint8_t* __restrict__ src, float* __restrict__ out,
                                                     int64_t nsuper, int nsb) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t sb = t >> 3;
    const int j = (int)(t & 7);
    if (sb >= nsuper) return;
    const int64_t n = sb / nsb;
    const int sidx = (int)(sb - n * nsb);
    uint4 h;
    h.x = *reinterpret_cast<const uint32_t*>(src + q4k_hdword(n, nsb, sidx, 0));
    h.y = *reinterpret_cast<const uint32_t*>(src + q4k_hdword(n, nsb, sidx, 1));
    h.z = *reinterpret_cast<const uint32_t*>(src + q4k_hdword(n, nsb, sidx, 2));
    h.w = *reinterpret_cast<const uint32_t*>(src + q4k_hdword(n, nsb, sidx, 3));
    const float d = q4k_hdr_d(h), dmin = q4k_hdr_dmin(h);
    uint32_t sc, m;
    q4k_hdr_sm(h, j, sc, m);
    const float d1 = d * (float)sc, m1 = dmin * (float)m;
    const int shift = (j & 1) * 4;
    float4* dst = reinterpret_cast<float4*>(out + sb * THQ_QK_K + 32 * j);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const uint4 v = *reinterpret_cast<const uint4*>(src + q4k_piece(n, nsb, sidx, hh, j >> 1));
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float4 o;
            o.x = d1 * (float)((w[i] >> shift) & 0xF) - m1;
            o.y = d1 * (float)((w[i] >> (shift + 8)) & 0xF) - m1;
            o.z = d1 * (float)((w[i] >> (shift + 16)) & 0xF) - m1;
            o.w = d1 * (float)((w[i] >> (shift + 24)) & 0xF) - m1;
            dst[4 * hh + i] = o;
        }
    }
}

// ---------------------------------------------------------------- Q4_K repack
// one thread per superblock: GGUF 144-B block -> row-quad layout
__global__ __launch_bounds__(256) void k_repack_q4k(const uint8_t* __restrict__ gguf, uint8_t* __restrict__ dst,
                                                    int64_t nsuper, int nsb) {
    const int64_t sb = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (sb >= nsuper) return;
    const int64_t n = sb / nsb;
    const int sidx = (int)(sb - n * nsb);
    const uint4* src = reinterpret_cast<const uint4*>(gguf + sb * THQ_Q4K_BYTES);
    const uint4 h = q4k_hdr_from_gguf(src[0]);
    const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
    for (int p = 0; p < 4; ++p) *reinterpret_cast<uint32_t*>(dst + q4k_hdword(n, nsb, sidx, p)) = hw[p];
#pragma unroll
    for (int c = 0; c < 8; ++c)  // 16-B chunk c of the nibbles = part c/2, half c%2
        *reinterpret_cast<uint4*>(dst + q4k_piece(n, nsb, sidx, c & 1, c >> 1)) = src[1 + c];
}

// one thread per (source row, superblock): copy between row-quad planes
__global__ __launch_bounds__(256) void k_q4k_copy_rows(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                       int64_t nsuper, int64_t dst_row0, int nsb) {
    const int64_t sb = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (sb >= nsuper) return;
    const int64_t n = sb / nsb;
    const int sidx = (int)(sb - n * nsb);
    const int64_t m = dst_row0 + n;
#pragma unroll
    for (int p = 0; p < 4; ++p)
        *reinterpret_cast<uint32_t*>(dst + q4k_hdword(m, nsb, sidx, p)) =
            *reinterpret_cast<const uint32_t*>(src + q4k_hdword(n, nsb, sidx, p));
#pragma unroll
    for (int c = 0; c < 8; ++c)
        *reinterpret_cast<uint4*>(dst + q4k_piece(m, nsb, sidx, c & 1, c >> 1)) =
            *reinterpret_cast<const uint4*>(src + q4k_piece(n, nsb, sidx, c & 1, c >> 1));
}

// ---------------------------------------------------------------- launchers
static inline unsigned grid_for(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

hipError_t launch_repack_q8_0(const uint8_t* raw, int8_t* qs, uint16_t* d, int64_t nblocks, hipStream_t s) {
    if (nblocks == 0) return hipSuccess;
    hipLaunchKernelGGL(k_repack_q8_0, dim3(grid_for(nblocks, 256)), dim3(256), 0, s, raw, qs, d, nblocks);
    return hipGetLastError();
}

hipError_t launch_quantize_q8_0(const float* w, int8_t* qs, uint16_t* d, int64_t nblocks, hipStream_t s) {
    if (nblocks == 0) return hipSuccess;
    hipLaunchKernelGGL(k_quantize_q8_0, dim3(grid_for(nblocks, 256)), dim3(256), 0, s, w, qs, d, nblocks);
    return hipGetLastError();
}

hipError_t launch_quantize_q4k(const float* w, uint8_t* dst, int64_t n, int nsb, hipStream_t s) {
    const int64_t nsuper = n * nsb;
    if (nsuper == 0) return hipSuccess;
    hipLaunchKernelGGL(k_quantize_q4k, dim3(grid_for(nsuper * 8, 256)), dim3(256), 0, s, w, dst, nsuper, nsb);
    return hipGetLastError();
}

hipError_t launch_repack_q4k(const uint8_t* gguf, uint8_t* dst, int64_t n, int nsb, hipStream_t s) {
    const int64_t nsuper = n * nsb;
    if (nsuper == 0) return hipSuccess;
    hipLaunchKernelGGL(k_repack_q4k, dim3(grid_for(nsuper, 256)), dim3(256), 0, s, gguf, dst, nsuper, nsb);
    return hipGetLastError();
}

hipError_t launch_q4k_copy_rows(const uint8_t* src, int64_t n, uint8_t* dst, int64_t dst_row0, int nsb,
                                hipStream_t s) {
    const int64_t nsuper = n * nsb;
    if (nsuper == 0) return hipSuccess;
    hipLaunchKernelGGL(k_q4k_copy_rows, dim3(grid_for(nsuper, 256)), dim3(256), 0, s, src, dst, nsuper, dst_row0,
                       nsb);
    return hipGetLastError();
}

hipError_t launch_dequant_q8_0(const int8_t* qs, const uint16_t* d, float* out, int64_t nblocks, hipStream_t s) {
    if (nblocks == 0) return hipSuccess;
    hipLaunchKernelGGL(k_dequant_q8_0, dim3(grid_for(nblocks, 256)), dim3(256), 0, s, qs, d, out, nblocks);
    return hipGetLastError();
}

hipError_t launch_dequant_q4k(const uint8_t* src, float* out, int64_t n, int nsb, hipStream_t s) {
    const int64_t nsuper = n * nsb;
    if (nsuper == 0) return hipSuccess;
    hipLaunchKernelGGL(k_dequant_q4k, dim3(grid_for(nsuper * 8, 256)), dim3(256), 0, s, src, out, nsuper, nsb);
    return hipGetLastError();
}

}  // namespace thq
