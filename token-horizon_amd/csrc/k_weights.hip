// k_weights.hip — weight preparation kernels for gfx950:
//   * repack GGUF Q8_0 blocks (34 B, 2-byte aligned) into the 32-row tile
//     layout (thq_dev.hpp, q8t_q / q8t_d); GGUF Q4_K blocks into the
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
// one thread per GGUF block b = row * nb + j: scale to the f16 plane, the two
// 16-B halves to the tile plane (thq_dev.hpp, q8t_q / q8t_d)
__global__ __launch_bounds__(256) void k_repack_q8_0(const uint8_t* __restrict__ raw, int8_t* __restrict__ qs,
                                                     uint16_t* __restrict__ dpl, int64_t nblocks, int64_t nb) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const int64_t row = b / nb, j = b - row * nb;
    const uint16_t* src = reinterpret_cast<const uint16_t*>(raw + b * THQ_Q8_0_BYTES);  // 2-B aligned
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = (uint32_t)src[1 + 2 * i] | ((uint32_t)src[2 + 2 * i] << 16);
    dpl[q8t_d(row, nb, j)] = src[0];
    *reinterpret_cast<uint4*>(qs + q8t_q(row, nb, j, 0)) = make_uint4(w[0], w[1], w[2], w[3]);
    *reinterpret_cast<uint4*>(qs + q8t_q(row, nb, j, 1)) = make_uint4(w[4], w[5], w[6], w[7]);
}

// ---------------------------------------------------------------- quantize Q8_0
__device__ __forceinline__ int8_t sat_i8(float v) {
    if (v != v) return 0;
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    return (int8_t)v;
}

__global__ __launch_bounds__(256) void k_quantize_q8_0(const float* __restrict__ w, int8_t* __restrict__ qs,
                                                       uint16_t* __restrict__ dpl, int64_t nblocks, int64_t nb) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const int64_t row = b / nb, j = b - row * nb;
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
    dpl[q8t_d(row, nb, j)] = dbits;
    uint32_t packed[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t v = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) v |= ((uint32_t)(uint8_t)sat_i8(roundf(x[4 * i + t] * id))) << (8 * t);
        packed[i] = v;
    }
    *reinterpret_cast<uint4*>(qs + q8t_q(row, nb, j, 0)) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    *reinterpret_cast<uint4*>(qs + q8t_q(row, nb, j, 1)) = make_uint4(packed[4], packed[5], packed[6], packed[7]);
}

// rows of one tile-layout Q8_0 weight into another (weight fusion): one
// thread per (source row, block)
__global__ __launch_bounds__(256) void k_q8_0_copy_rows(const int8_t* __restrict__ sq, const uint16_t* __restrict__ sd,
                                                        int64_t nsrc, int8_t* __restrict__ dq, uint16_t* __restrict__ dd,
                                                        int64_t row0, int64_t nb) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nsrc * nb) return;
    const int64_t row = b / nb, j = b - row * nb;
    dd[q8t_d(row0 + row, nb, j)] = sd[q8t_d(row, nb, j)];
#pragma unroll
    for (int g = 0; g < 2; ++g)
        *reinterpret_cast<uint4*>(dq + q8t_q(row0 + row, nb, j, g)) =
            *reinterpret_cast<const uint4*>(sq + q8t_q(row, nb, j, g));
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
// four outputs: f32, or bf16 rounded to nearest even from the f32 values
__device__ __forceinline__ void put4(float* p, float a, float b, float c, float d) {
    *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
}
__device__ __forceinline__ void put4(bf16_t* p, float a, float b, float c, float d) {
    *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(a, b), pack_bf16x2(c, d));
}

// one thread per 32-weight block: y = q * d
template <typename OT>
__global__ __launch_bounds__(256) void k_dequant_q8_0(const int8_t* __restrict__ qs,
                                                      const uint16_t* __restrict__ dpl, OT* __restrict__ out,
                                                      int64_t nblocks, int64_t nb) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const int64_t row = b / nb, j = b - row * nb;
    const float d = f16_to_f32(dpl[q8t_d(row, nb, j)]);
    OT* dst = out + b * THQ_QK8_0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint4 v = *reinterpret_cast<const uint4*>(qs + q8t_q(row, nb, j, h));
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
            put4(dst + 16 * h + 4 * i, (float)(int8_t)(w[i] & 0xFF) * d, (float)(int8_t)((w[i] >> 8) & 0xFF) * d,
                 (float)(int8_t)((w[i] >> 16) & 0xFF) * d, (float)(int8_t)(w[i] >> 24) * d);
    }
}

// bf16 output: one wave per (row, 2048-weight chunk of K), eight rows per
// block (a tile record's 128-B lines hold eight rows).  Store instruction i
// of a wave writes weights 512 i + 8 lane .. + 7 of the chunk: 1 KB
// contiguous.  A lane loads the 8-B half of its block's 16-B piece and the
// block's scale.  Values as k_dequant_q8_0.
__global__ __launch_bounds__(512) void k_dequant_q8_0_b16(const int8_t* __restrict__ qs,
                                                          const uint16_t* __restrict__ dpl, bf16_t* __restrict__ out,
                                                          int64_t n, int64_t nb, int64_t nchunks) {
    const int lane = threadIdx.x & 63;
    const int64_t grp = (int64_t)blockIdx.x / nchunks, chunk = (int64_t)blockIdx.x - grp * nchunks;
    const int64_t row = grp * 8 + (threadIdx.x >> 6);
    if (row >= n) return;
    const int64_t K = nb * 32;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t k = chunk * 2048 + 512 * i + 8 * lane;
        if (k < K) {
            const int64_t b = k >> 5;
            const int off = (int)(k & 31);  // 0, 8, 16, 24: half (off & 8) of piece off / 16
            const float d = f16_to_f32(dpl[q8t_d(row, nb, b)]);
            const uint2 v = *reinterpret_cast<const uint2*>(qs + q8t_q(row, nb, b, off >> 4) + (off & 8));
            const uint32_t w[2] = {v.x, v.y};
            uint32_t o[4];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                o[2 * t] = pack_bf16x2((float)(int8_t)(w[t] & 0xFF) * d, (float)(int8_t)((w[t] >> 8) & 0xFF) * d);
                o[2 * t + 1] = pack_bf16x2((float)(int8_t)((w[t] >> 16) & 0xFF) * d, (float)(int8_t)(w[t] >> 24) * d);
            }
            *reinterpret_cast<uint4*>(out + row * K + k) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
}

// one thread per (superblock, sub-block j): y = d*sc*q - dmin*m
template <typename OT>
__global__ __launch_bounds__(256) void k_dequant_q4k(const uint8_t* __restrict__ src, OT* __restrict__ out,
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
    OT* dst = out + sb * THQ_QK_K + 32 * j;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const uint4 v = *reinterpret_cast<const uint4*>(src + q4k_piece(n, nsb, sidx, hh, j >> 1));
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
            put4(dst + 16 * hh + 4 * i, d1 * (float)((w[i] >> shift) & 0xF) - m1,
                 d1 * (float)((w[i] >> (shift + 8)) & 0xF) - m1, d1 * (float)((w[i] >> (shift + 16)) & 0xF) - m1,
                 d1 * (float)((w[i] >> (shift + 24)) & 0xF) - m1);
    }
}

// ---------------------------------------------------------------- Q6_K
// GGUF 210-B blocks (2-B aligned) -> planes regrouped by 64-weight step
// (thq_dev.hpp, q6k_layout); one thread per superblock
__global__ __launch_bounds__(256) void k_repack_q6k(const uint8_t* __restrict__ gguf, uint8_t* __restrict__ dst,
                                                    int64_t n, int nsb) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n * nsb) return;
    const int64_t row = b / nsb;
    const int s = (int)(b - row * nsb);
    const int64_t K = (int64_t)nsb * 256;
    const Q6Layout L = q6k_layout(n, K);
    const uint16_t* src = reinterpret_cast<const uint16_t*>(gguf + b * 210);
    uint32_t w[52];
#pragma unroll
    for (int i = 0; i < 52; ++i) w[i] = (uint32_t)src[2 * i] | ((uint32_t)src[2 * i + 1] << 16);
    const uint32_t* ql = w;        // ql[128]
    const uint32_t* qh = w + 32;   // qh[64]
    uint32_t* qlo = reinterpret_cast<uint32_t*>(dst + row * (K / 2) + s * 128);
    uint32_t* qho = reinterpret_cast<uint32_t*>(dst + L.qh + row * (K / 4) + s * 64);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        // QL: step 2h takes the low nibbles of ql[64h + t] (weight t) and
        // ql[64h + 32 + t] (weight t + 32), step 2h + 1 the high nibbles
#pragma unroll
        for (int t4 = 0; t4 < 8; ++t4) {
            const uint32_t a = ql[16 * h + t4], c = ql[16 * h + 8 + t4];
            qlo[16 * h + t4] = (a & 0x0F0F0F0Fu) | ((c & 0x0F0F0F0Fu) << 4);
            qlo[16 * h + 8 + t4] = ((a >> 4) & 0x0F0F0F0Fu) | (c & 0xF0F0F0F0u);
        }
        // QH: step weight w of step 2h + e sits in quarter 2e + w/32 at l = w % 32,
        // i.e. in bits 2(2e + w/32) of qh[32h + w % 32]; byte t collects w = t,
        // t + 16, t + 32, t + 48
#pragma unroll
        for (int e = 0; e < 2; ++e) {
#pragma unroll
            for (int t4 = 0; t4 < 4; ++t4) {
                const uint32_t lo = qh[8 * h + t4], hi = qh[8 * h + 4 + t4];  // qh[32h + 4t4 ..], qh[32h + 16 + 4t4 ..]
                const int s0 = 4 * e, s1 = 4 * e + 2;
                const uint32_t v = ((lo >> s0) & 0x03030303u) | (((hi >> s0) & 0x03030303u) << 2) |
                                   (((lo >> s1) & 0x03030303u) << 4) | (((hi >> s1) & 0x03030303u) << 6);
                qho[8 * h + 4 * e + t4] = v;
            }
        }
    }
    uint4* sc = reinterpret_cast<uint4*>(dst + L.sc + row * (K / 16) + s * 16);
    sc[0] = make_uint4(w[48], w[49], w[50], w[51]);
    reinterpret_cast<uint16_t*>(dst + L.d)[row * nsb + s] = src[104];
}

// one thread per (row, 64-weight step): w = (d * sc) * (code - 32), GGML's order
template <typename OT>
__global__ __launch_bounds__(256) void k_dequant_q6k(const uint8_t* __restrict__ src, OT* __restrict__ out, int64_t n,
                                                     int nsb) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n * nsb * 4) return;
    const int64_t row = t / (4 * nsb);
    const int j = (int)(t - row * 4 * nsb);  // step index in the row
    const int64_t K = (int64_t)nsb * 256;
    const Q6Layout L = q6k_layout(n, K);
    const uint8_t* ql = src + row * (K / 2) + j * 32;
    const uint8_t* qh = src + L.qh + row * (K / 4) + j * 16;
    const int8_t* sc = reinterpret_cast<const int8_t*>(src + L.sc + row * (K / 16) + j * 4);
    const float d = f16_to_f32(reinterpret_cast<const uint16_t*>(src + L.d)[row * nsb + (j >> 2)]);
    OT* y = out + row * K + j * 64;
    for (int w0 = 0; w0 < 64; w0 += 4) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int w = w0 + i;
            const int code = ((ql[w & 31] >> (4 * (w >> 5))) & 0xF) | (((qh[w & 15] >> (2 * (w >> 4))) & 3) << 4);
            v[i] = d * (float)sc[w >> 4] * (float)(code - 32);
        }
        put4(y + w0, v[0], v[1], v[2], v[3]);
    }
}

// bf16 output: one lane per 16 weights 16u .. 16u + 15 of a 64-weight step
// (4 lanes per step): their low four bits are ql bytes 16 (u & 1) .. + 15 of
// the step (nibble u >> 1), their high two bits the step's 16 qh bytes (bits
// 2u, 2u + 1), their scale sc[u]; two 16-B loads, two 16-B stores.  Values
// as k_dequant_q6k: d * sc * (code - 32) in f32, then bf16 to nearest even.
__global__ __launch_bounds__(256) void k_dequant_q6k_b16(const uint8_t* __restrict__ src, bf16_t* __restrict__ out,
                                                         int64_t n, int nsb) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t step = t >> 2;
    if (step >= n * nsb * 4) return;
    const int u = (int)t & 3;
    const int64_t row = step / (4 * nsb);
    const int j = (int)(step - row * 4 * nsb);
    const int64_t K = (int64_t)nsb * 256;
    const Q6Layout L = q6k_layout(n, K);
    const uint4 ql = *reinterpret_cast<const uint4*>(src + row * (K / 2) + j * 32 + 16 * (u & 1));
    const uint4 qh = *reinterpret_cast<const uint4*>(src + L.qh + row * (K / 4) + j * 16);
    const float sc = (float)reinterpret_cast<const int8_t*>(src + L.sc + row * (K / 16) + j * 4)[u];
    const float d = f16_to_f32(reinterpret_cast<const uint16_t*>(src + L.d)[row * nsb + (j >> 2)]);
    const float ds = d * sc;
    const uint32_t l4[4] = {ql.x, ql.y, ql.z, ql.w}, h4[4] = {qh.x, qh.y, qh.z, qh.w};
    const int sl = 4 * (u >> 1), sh = 2 * u;
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // four 6-bit codes, one per byte
        const uint32_t c = ((l4[i] >> sl) & 0x0F0F0F0Fu) | (((h4[i] >> sh) & 0x03030303u) << 4);
        o[2 * i] = pack_bf16x2(ds * (float)((int)(c & 0xFF) - 32), ds * (float)((int)((c >> 8) & 0xFF) - 32));
        o[2 * i + 1] = pack_bf16x2(ds * (float)((int)((c >> 16) & 0xFF) - 32), ds * (float)((int)(c >> 24) - 32));
    }
    uint4* dst = reinterpret_cast<uint4*>(out + row * K + j * 64 + 16 * u);
    dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
    dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
}

// ---------------------------------------------------------------- MLX affine 4-bit
// half 2.7.1 bf16::from_f64 (its f64_to_bf16, the rounding dequant_affine
// uses, engine/src/qwen35.rs:110-134): the low 32 bits of the f64 mantissa
// are dropped first, then the top 20 mantissa bits round to nearest even
// (the round bit decides, the remaining kept bits and the result's last bit
// break ties), with half's overflow, subnormal and NaN rules.
__device__ __forceinline__ uint16_t bf16_from_f64_half(double v) {
    const uint32_t x = (uint32_t)((uint64_t)__double_as_longlong(v) >> 32);
    const uint32_t sign = x & 0x80000000u, exp = x & 0x7FF00000u;
    uint32_t man = x & 0x000FFFFFu;
    const uint32_t hs = sign >> 16;
    if (exp == 0x7FF00000u) {  // inf / NaN (NaN keeps the top mantissa bits, quiet bit set)
        const uint32_t nan_bit = (man == 0 && (uint32_t)__double_as_longlong(v) == 0) ? 0u : 0x0040u;
        return (uint16_t)(hs | 0x7F80u | nan_bit | (man >> 13));
    }
    const int he = (int)(exp >> 20) - 1023 + 127;
    if (he >= 0xFF) return (uint16_t)(hs | 0x7F80u);
    if (he <= 0) {
        if (14 - he > 21) return (uint16_t)hs;  // the round bit lies above the hidden bit
        man |= 0x00100000u;
        uint32_t hm = man >> (14 - he);
        const uint32_t rb = 1u << (13 - he);
        if ((man & rb) && (man & (3u * rb - 1u))) hm += 1;
        return (uint16_t)(hs | hm);
    }
    const uint32_t r = hs | ((uint32_t)he << 7) | (man >> 13);
    return (uint16_t)(((man & 0x1000u) && (man & 0x2FFFu)) ? r + 1 : r);
}

// The same rounding where the value is +-0 or its 20-mantissa-bit truncation
// lies in the normal bf16 range: that truncation is exact in f32, and the
// f32 -> bf16 round to nearest even (v_cvt_pk_bf16_f32) then sees the same
// round bit (mantissa bit 12), sticky bits (11..0) and last kept bit (13) as
// the rule above.  Returns false, with f unused, for subnormal, overflowing,
// infinite and NaN values.
__device__ __forceinline__ bool f64_half_fast(double v, float& f) {
    const uint64_t b = (uint64_t)__double_as_longlong(v) & 0xFFFFFFFF00000000ull;
    const uint32_t e = (uint32_t)(b >> 52) & 0x7FFu;
    f = (float)__longlong_as_double((long long)b);
    return (e >= 1023 - 126 && e <= 1023 + 127) || (b << 1) == 0;
}

// MLX affine -> row-quad plane.  One thread per (row, 64-weight part of the
// padded K): the part's eight words (element e = nibble e%8 of word e/8,
// LSB first) become the two 16-B pieces (byte i: low = element i, high =
// element 32 + i, i = 16h + j) and the header dword (bf16 scale | bf16 bias
// << 16) of the group the part belongs to; parts past K are zero.
// Source layouts (the engine's QLin, engine/src/qwen35.rs:311-319):
//   row-major  wq [n][K/8], sb [n][2*ng]: the row's ng = K/gs scales, then
//              its ng biases
//   tiled      QLin::tiled (qwen35.rs:629-697), addresses q4woff / q4sb of
//              engine/src/quant_kernel.rs:1085-1101: wq [row/256][g][row%256][8],
//              scales [(tile*ng + g)*256 + row%256], biases after all
//              tiles*ng*256 scales (gs = 64)
__global__ __launch_bounds__(256) void k_repack_affine(const uint32_t* __restrict__ wq,
                                                       const uint16_t* __restrict__ sb, uint8_t* __restrict__ dst,
                                                       int64_t n, int K, int gs, int tiled, int nsb) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int nparts = nsb * 4;
    if (t >= n * nparts) return;
    const int64_t row = t / nparts;
    const int gp = (int)(t - row * nparts);
    const int s = gp >> 2, p = gp & 3;
    uint32_t pc[2][4] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
    uint32_t hw = 0;
    const int ng64 = K >> 6;
    if (gp < ng64) {
        const int64_t base = tiled ? (row >> 8) * (int64_t)ng64 * 2048 + (int64_t)gp * 2048 + (row & 255) * 8
                                   : row * (int64_t)(K >> 3) + (int64_t)gp * 8;
        uint32_t wd[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) wd[i] = wq[base + i];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint32_t lo = (wd[2 * h + (j >> 3)] >> (4 * (j & 7))) & 0xFu;
                const uint32_t hi = (wd[4 + 2 * h + (j >> 3)] >> (4 * (j & 7))) & 0xFu;
                pc[h][j >> 2] |= (lo | (hi << 4)) << (8 * (j & 3));
            }
        uint32_t sc, bi;
        if (tiled) {
            const int64_t tiles = (n + 255) >> 8;
            const int64_t prm = ((row >> 8) * ng64 + gp) * 256 + (row & 255);
            sc = sb[prm];
            bi = sb[prm + tiles * ng64 * 256];
        } else {
            const int ng = K / gs, g = gp * 64 / gs;
            sc = sb[row * 2 * ng + g];
            bi = sb[row * 2 * ng + ng + g];
        }
        hw = sc | (bi << 16);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
        *reinterpret_cast<uint4*>(dst + q4k_piece(row, nsb, s, h, p)) = make_uint4(pc[h][0], pc[h][1], pc[h][2], pc[h][3]);
    *reinterpret_cast<uint32_t*>(dst + q4k_hdword(row, nsb, s, p)) = hw;
}

// One thread per (row, 64-weight group): out = fmaf(q, scale, bias) (the
// product is exact, so one rounding of q*scale + bias).
__global__ __launch_bounds__(256) void k_dequant_affine(const uint8_t* __restrict__ src, float* __restrict__ out,
                                                        int64_t n, int K, int nsb) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int ng64 = K >> 6;
    if (t >= n * ng64) return;
    const int64_t row = t / ng64;
    const int gp = (int)(t - row * ng64);
    const int s = gp >> 2, p = gp & 3;
    const uint32_t hw = *reinterpret_cast<const uint32_t*>(src + q4k_hdword(row, nsb, s, p));
    const float sc = aff_scale(hw), bi = aff_bias(hw);
    float* of = out + row * (int64_t)K + 64 * gp;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint4 v = *reinterpret_cast<const uint4*>(src + q4k_piece(row, nsb, s, h, p));
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int half = 0; half < 2; ++half) {  // low nibbles: elements 16h + j; high: 32 + 16h + j
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float q[4];
#pragma unroll
                for (int b = 0; b < 4; ++b) q[b] = (float)((w[i] >> (8 * b + 4 * half)) & 0xFu);
                put4(of + 32 * half + 16 * h + 4 * i, __builtin_fmaf(q[0], sc, bi), __builtin_fmaf(q[1], sc, bi),
                     __builtin_fmaf(q[2], sc, bi), __builtin_fmaf(q[3], sc, bi));
            }
        }
    }
}

// bf16 output of the row-quad layout (Q4_K and MLX affine: the dequantize-
// then-GEMM route writes 2 B per weight, 3.6x the bytes it reads).  One lane
// per 8-byte half k of a 16-B nibble piece (h, s, p), 4 lanes per 64-weight
// group: the half's low nibbles are elements 64 gp + 16h + 8k .. + 7 of the
// row (gp = 4s + p) and its high nibbles the same + 32, so each lane makes
// two 16-B stores and a group's four lanes fill each 64-B run of the output
// in one store instruction.  Q4_K: d1 * q - m1 in f32 (as k_dequant_q4k),
// then bf16 to nearest even; affine: half's f64 -> bf16 of q * scale + bias
// evaluated in f64, as dequant_affine does.
template <bool AFF>
__global__ __launch_bounds__(256) void k_dequant_q4_b16(const uint8_t* __restrict__ src, bf16_t* __restrict__ out,
                                                        int64_t n, int K, int nsb) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int ng64 = K >> 6;
    const int64_t grp = t >> 2;
    if (grp >= n * ng64) return;
    const int64_t row = grp / ng64;
    const int gp = (int)(grp - row * ng64);
    const int s = gp >> 2, p = gp & 3, h = (int)(t >> 1) & 1, k = (int)t & 1;
    const uint2 v = *reinterpret_cast<const uint2*>(src + q4k_piece(row, nsb, s, h, p) + 8 * k);
    const uint32_t w[2] = {v.x, v.y};
    uint32_t lo[4], hi[4];
    if constexpr (AFF) {
        const uint32_t hw = *reinterpret_cast<const uint32_t*>(src + q4k_hdword(row, nsb, s, p));
        const double sc = (double)aff_scale(hw), bi = (double)aff_bias(hw);
        // element e's code: lo half e < 8 from byte e, hi half from its high nibble
        double v[16];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t byte = (w[e >> 2] >> (8 * (e & 3))) & 0xFFu;
            v[e] = (double)(float)(byte & 0xF) * sc + bi;
            v[8 + e] = (double)(float)(byte >> 4) * sc + bi;
        }
        float f[16];
        bool fast = true;
#pragma unroll
        for (int e = 0; e < 16; ++e) fast = f64_half_fast(v[e], f[e]) && fast;
        uint32_t o[8];
        if (fast) {
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                o[i] = (uint32_t)bf16_from_f64_half(v[2 * i]) | ((uint32_t)bf16_from_f64_half(v[2 * i + 1]) << 16);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lo[i] = o[i];
            hi[i] = o[4 + i];
        }
    } else {
        uint4 hd;
        hd.x = *reinterpret_cast<const uint32_t*>(src + q4k_hdword(row, nsb, s, 0));
        hd.y = *reinterpret_cast<const uint32_t*>(src + q4k_hdword(row, nsb, s, 1));
        hd.z = *reinterpret_cast<const uint32_t*>(src + q4k_hdword(row, nsb, s, 2));
        hd.w = *reinterpret_cast<const uint32_t*>(src + q4k_hdword(row, nsb, s, 3));
        const float d = q4k_hdr_d(hd), dmin = q4k_hdr_dmin(hd);
        uint32_t sc0, m0, sc1, m1;
        q4k_hdr_sm(hd, 2 * p, sc0, m0);
        q4k_hdr_sm(hd, 2 * p + 1, sc1, m1);
        const float dl = d * (float)sc0, ml = dmin * (float)m0;
        const float dh = d * (float)sc1, mh = dmin * (float)m1;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t x = w[i];
            lo[2 * i] = pack_bf16x2(dl * (float)(x & 0xF) - ml, dl * (float)((x >> 8) & 0xF) - ml);
            lo[2 * i + 1] = pack_bf16x2(dl * (float)((x >> 16) & 0xF) - ml, dl * (float)((x >> 24) & 0xF) - ml);
            hi[2 * i] = pack_bf16x2(dh * (float)((x >> 4) & 0xF) - mh, dh * (float)((x >> 12) & 0xF) - mh);
            hi[2 * i + 1] = pack_bf16x2(dh * (float)((x >> 20) & 0xF) - mh, dh * (float)(x >> 28) - mh);
        }
    }
    bf16_t* dst = out + row * (int64_t)K + 64 * gp + 16 * h + 8 * k;
    *reinterpret_cast<uint4*>(dst) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    *reinterpret_cast<uint4*>(dst + 32) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
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

hipError_t launch_repack_q8_0(const uint8_t* raw, int8_t* qs, uint16_t* d, int64_t n, int64_t nb, hipStream_t s) {
    const int64_t nblocks = n * nb;
    if (nblocks == 0) return hipSuccess;
    hipLaunchKernelGGL(k_repack_q8_0, dim3(grid_for(nblocks, 256)), dim3(256), 0, s, raw, qs, d, nblocks, nb);
    return hipGetLastError();
}

hipError_t launch_quantize_q8_0(const float* w, int8_t* qs, uint16_t* d, int64_t n, int64_t nb, hipStream_t s) {
    const int64_t nblocks = n * nb;
    if (nblocks == 0) return hipSuccess;
    hipLaunchKernelGGL(k_quantize_q8_0, dim3(grid_for(nblocks, 256)), dim3(256), 0, s, w, qs, d, nblocks, nb);
    return hipGetLastError();
}

hipError_t launch_q8_0_copy_rows(const int8_t* sq, const uint16_t* sd, int64_t nsrc, int8_t* dq, uint16_t* dd,
                                 int64_t row0, int64_t nb, hipStream_t s) {
    if (nsrc * nb == 0) return hipSuccess;
    hipLaunchKernelGGL(k_q8_0_copy_rows, dim3(grid_for(nsrc * nb, 256)), dim3(256), 0, s, sq, sd, nsrc, dq, dd, row0,
                       nb);
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

hipError_t launch_dequant_q8_0(const int8_t* qs, const uint16_t* d, void* out, bool bf16, int64_t n, int64_t nb,
                               hipStream_t s) {
    const int64_t nblocks = n * nb;
    if (nblocks == 0) return hipSuccess;
    if (bf16) {
        const int64_t nchunks = (nb * 32 + 2047) / 2048, blocks = (n + 7) / 8 * nchunks;
        if (blocks >= (1ll << 31)) return hipErrorInvalidValue;
        hipLaunchKernelGGL(k_dequant_q8_0_b16, dim3((unsigned)blocks), dim3(512), 0, s, qs, d,
                           static_cast<bf16_t*>(out), n, nb, nchunks);
    } else {
        hipLaunchKernelGGL(k_dequant_q8_0<float>, dim3(grid_for(nblocks, 256)), dim3(256), 0, s, qs, d,
                           static_cast<float*>(out), nblocks, nb);
    }
    return hipGetLastError();
}

hipError_t launch_dequant_q4k(const uint8_t* src, void* out, bool bf16, int64_t n, int nsb, hipStream_t s) {
    const int64_t nsuper = n * nsb;
    if (nsuper == 0) return hipSuccess;
    if (bf16)
        hipLaunchKernelGGL(k_dequant_q4_b16<false>, dim3(grid_for(nsuper * 16, 256)), dim3(256), 0, s, src,
                           static_cast<bf16_t*>(out), n, nsb * 256, nsb);
    else
        hipLaunchKernelGGL(k_dequant_q4k<float>, dim3(grid_for(nsuper * 8, 256)), dim3(256), 0, s, src,
                           static_cast<float*>(out), nsuper, nsb);
    return hipGetLastError();
}

hipError_t launch_repack_q6k(const uint8_t* gguf, uint8_t* dst, int64_t n, int nsb, hipStream_t s) {
    if (n * nsb == 0) return hipSuccess;
    hipLaunchKernelGGL(k_repack_q6k, dim3(grid_for(n * nsb, 256)), dim3(256), 0, s, gguf, dst, n, nsb);
    return hipGetLastError();
}

hipError_t launch_dequant_q6k(const uint8_t* src, void* out, bool bf16, int64_t n, int nsb, hipStream_t s) {
    const int64_t t = n * nsb * 4;
    if (t == 0) return hipSuccess;
    if (bf16)
        hipLaunchKernelGGL(k_dequant_q6k_b16, dim3(grid_for(t * 4, 256)), dim3(256), 0, s, src,
                           static_cast<bf16_t*>(out), n, nsb);
    else
        hipLaunchKernelGGL(k_dequant_q6k<float>, dim3(grid_for(t, 256)), dim3(256), 0, s, src, static_cast<float*>(out),
                           n, nsb);
    return hipGetLastError();
}

hipError_t launch_repack_affine(const uint32_t* wq, const uint16_t* sb, uint8_t* dst, int64_t n, int K, int gs,
                                bool tiled, hipStream_t s) {
    const int nsb = (K + 255) / 256;
    const int64_t threads = n * nsb * 4;
    if (threads == 0) return hipSuccess;
    hipLaunchKernelGGL(k_repack_affine, dim3(grid_for(threads, 256)), dim3(256), 0, s, wq, sb, dst, n, K, gs,
                       tiled ? 1 : 0, nsb);
    return hipGetLastError();
}

hipError_t launch_dequant_affine(const uint8_t* src, void* out, bool bf16, int64_t n, int K, hipStream_t s) {
    const int nsb = (K + 255) / 256;
    const int64_t threads = n * (K / 64);
    if (threads == 0) return hipSuccess;
    if (bf16)
        hipLaunchKernelGGL(k_dequant_q4_b16<true>, dim3(grid_for(threads * 4, 256)), dim3(256), 0, s, src,
                           static_cast<bf16_t*>(out), n, K, nsb);
    else
        hipLaunchKernelGGL(k_dequant_affine, dim3(grid_for(threads, 256)), dim3(256), 0, s, src,
                           static_cast<float*>(out), n, K, nsb);
    return hipGetLastError();
}

}  // namespace thq
