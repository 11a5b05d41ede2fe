// thq_dev.hpp — device-side helpers shared by the gfx950 kernels.
//
// Block formats (GGML, as candle-core's k_quants stores them):
//   Q8_0: 32 weights / 34 B  = f16 d, i8 qs[32]            (repacked on device
//         into an i8 plane [N][K] and an f16 scale plane [N][K/32])
//   Q4_K: 256 weights / 144 B = f16 d, f16 dmin, u8 scales[12], u8 qs[128]
//         (kept in GGUF order: one 144-B superblock is nine 16-B vectors)
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define THQ_QK8_0 32
#define THQ_QK_K 256
#define THQ_Q4K_BYTES 144
#define THQ_Q8_0_BYTES 34

typedef uint16_t bf16_t;  // raw bf16 bits
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace thq {

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;  // exact
}

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// round to nearest even (v_cvt_pk_bf16_f32 on gfx950)
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
    __bf16 b = (__bf16)f;
    bf16_t r;
    __builtin_memcpy(&r, &b, 2);
    return r;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// GGML get_scale_min_k4 on the 12 scale bytes held as three dwords
// s0 = scales[0..3], s1 = scales[4..7], s2 = scales[8..11].
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t& sc,
                                             uint32_t& m) {
    if (j < 4) {
        sc = (s0 >> (8 * j)) & 63u;
        m = (s1 >> (8 * j)) & 63u;
    } else {
        const int i = j - 4;
        const uint32_t b8 = (s2 >> (8 * i)) & 0xFFu;  // scales[j+4]
        sc = (b8 & 0xFu) | (((s0 >> (8 * i + 6)) & 3u) << 4);
        m = (b8 >> 4) | (((s1 >> (8 * i + 6)) & 3u) << 4);
    }
}

// byte I of w as f32 (selected to v_cvt_f32_ubyteI)
template <int I>
__device__ __forceinline__ float ubyte_f32(uint32_t w) {
    return (float)((w >> (8 * I)) & 0xFFu);
}

// 64-lane sum; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

template <typename YT>
__device__ __forceinline__ void store_y(YT* p, float v);
template <>
__device__ __forceinline__ void store_y<float>(float* p, float v) {
    *p = v;
}
template <>
__device__ __forceinline__ void store_y<bf16_t>(bf16_t* p, float v) {
    *p = f32_to_bf16(v);
}

template <typename XT>
__device__ __forceinline__ float load_x(const XT* p);
template <>
__device__ __forceinline__ float load_x<float>(const float* p) {
    return *p;
}
template <>
__device__ __forceinline__ float load_x<bf16_t>(const bf16_t* p) {
    return bf16_to_f32(*p);
}

// silu(bf16(g)) * bf16(u) in f32, the reference kernel's epilogue form.
__device__ __forceinline__ float silu_mul(float g, float u) {
    const float gb = bf16_round(g);
    const float ub = bf16_round(u);
    return gb / (1.0f + expf(-gb)) * ub;
}

}  // namespace thq
