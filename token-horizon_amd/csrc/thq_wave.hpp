// thq_wave.hpp — wave-level helpers shared by the M = 1 GEMV kernels: bf16
// pair dots, per-wave row slots and the cross-lane reductions of per-row
// partial sums (DPP within 16-lane rows, shuffles across them).
#pragma once

#include "thq_dev.hpp"

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

// ------------------------------------------------------------------ wave helpers
// value of lane P of each quad, in every lane of the quad (DPP quad_perm)
template <int P>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, P | (P << 2) | (P << 4) | (P << 6), 0xF, 0xF, false);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

// sum over the 16 lanes of each DPP row; every lane of the row gets it
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    v += dpp_f<0x140>(v);  // row_mirror
    return v;
}

// Transposed reduction of R per-lane partials over the 64 lanes: each step
// halves the values a lane carries, so R rows cost about as much as one.
// Afterwards every lane holds the total of slot slot_of_lane<R>(lane): R=1
// slot 0 everywhere; R=2 slot lane/32; R=4 slot 2*(lane/32) + (lane/16)%2.
template <int R>
__device__ __forceinline__ float reduce_slots(const float (&v)[R], int lane) {
    const bool up = lane & 32, b4 = lane & 16;
    float k;
    if constexpr (R == 4) {
        const float s0 = up ? v[0] : v[2], s1 = up ? v[1] : v[3];
        const float k0 = (up ? v[2] : v[0]) + __shfl_xor(s0, 32, 64);
        const float k1 = (up ? v[3] : v[1]) + __shfl_xor(s1, 32, 64);
        k = (b4 ? k1 : k0) + __shfl_xor(b4 ? k0 : k1, 16, 64);
    } else if constexpr (R == 2) {
        k = (up ? v[1] : v[0]) + __shfl_xor(up ? v[0] : v[1], 32, 64);
        k += __shfl_xor(k, 16, 64);
    } else {
        k = v[0] + __shfl_xor(v[0], 32, 64);
        k += __shfl_xor(k, 16, 64);
    }
    return row16_sum(k);
}

template <int R>
__device__ __forceinline__ int slot_of_lane(int lane) {
    if constexpr (R == 4) return 2 * (lane >> 5) + ((lane >> 4) & 1);
    if constexpr (R == 2) return lane >> 5;
    return 0;
}

// Argmax combine of (value, index) pairs across lanes: larger value, else
// lower index.  With NaN entered as -inf and every lane holding its own
// output's index, a butterfly over W lanes equals the strict '>' scan from
// (-inf, lowest index) over those outputs: NaN is never chosen, and a group
// of -inf / NaN only yields its lowest index.
__device__ __forceinline__ float amax_key(float v) { return v != v ? -INFINITY : v; }

template <int CTRL>
__device__ __forceinline__ void amax_dpp(float& v, uint32_t& i) {
    const float v2 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
    const uint32_t i2 = (uint32_t)__builtin_amdgcn_mov_dpp((int)i, CTRL, 0xF, 0xF, false);
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

// combine over each 16-lane DPP row (the pairings of row16_sum); every lane
// of the row ends with the row's (max, lowest index)
__device__ __forceinline__ void amax_row16(float& v, uint32_t& i) {
    amax_dpp<0xB1>(v, i);   // quad_perm [1,0,3,2]
    amax_dpp<0x4E>(v, i);   // quad_perm [2,3,0,1]
    amax_dpp<0x141>(v, i);  // row_half_mirror
    amax_dpp<0x140>(v, i);  // row_mirror
}

// the same over 32 lanes (two rows, then one exchange across them)
__device__ __forceinline__ void amax_row32(float& v, uint32_t& i) {
    amax_row16(v, i);
    const float v2 = __shfl_xor(v, 16, 64);
    const uint32_t i2 = __shfl_xor(i, 16, 64);
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

}  // namespace thq
