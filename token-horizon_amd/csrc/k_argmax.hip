// k_argmax.hip — per-row greedy argmax over f32 logits.
//
// Tie rule of engine/src/engine.rs:1891-1898 (greedy_argmax) and candle's
// arg-reduce: a strict '>' scan from (index 0, -inf), so the lowest index
// among equal maxima wins, NaN is never selected and a row of -inf gives 0.
// Two passes: chunks of 2048 elements per block, then one block per row over
// the chunk partials.  The combine (larger value, else lower index) is
// associative, so the result equals the sequential scan's.
#include "thq_dev.hpp"
#include "thq_kernels.hpp"

namespace thq {

__device__ __forceinline__ void amax_combine(float& v, uint32_t& i, float v2, uint32_t i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

// block combine (up to 1024 threads); thread 0 ends with the result
__device__ __forceinline__ void block_amax(float& v, uint32_t& i) {
    __shared__ float sv[16];
    __shared__ uint32_t si[16];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float v2 = __shfl_xor(v, off, 64);
        const uint32_t i2 = __shfl_xor(i, off, 64);
        amax_combine(v, i, v2, i2);
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[wave] = v;
        si[wave] = i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) amax_combine(v, i, sv[w], si[w]);
    }
}

// pass 1: grid (chunks, M).  Each thread takes 8 entries 256 apart, loaded
// independently (the pass is latency-bound: one dependent load per step left
// a single block per row waiting on memory ~40 times), then the block
// combine.  Values: index = position, NaN enters as -inf; pairs: the fused
// epilogues' (max, index) partials.  Absent entries are (-inf, UINT32_MAX),
// which never win.
constexpr int AMAX_PT = 8;
constexpr int AMAX_CHUNK = 256 * AMAX_PT;

template <bool PAIRS>
__global__ __launch_bounds__(256) void k_amax_pass(const float* __restrict__ v, const uint32_t* __restrict__ iv,
                                                   int64_t n, int64_t ld, int chunks, float* __restrict__ pv,
                                                   uint32_t* __restrict__ pi) {
    const int64_t row = blockIdx.y;
    const int64_t c0 = (int64_t)blockIdx.x * AMAX_CHUNK + threadIdx.x;
    float vals[AMAX_PT];
    uint32_t ids[AMAX_PT];
#pragma unroll
    for (int j = 0; j < AMAX_PT; ++j) {
        const int64_t k = c0 + (int64_t)j * 256;
        const bool in = k < n;
        const float x = in ? v[row * ld + k] : -INFINITY;
        vals[j] = x != x ? -INFINITY : x;
        ids[j] = in ? (PAIRS ? iv[row * ld + k] : (uint32_t)k) : 0xFFFFFFFFu;
    }
    float bv = vals[0];
    uint32_t bi = ids[0];
#pragma unroll
    for (int j = 1; j < AMAX_PT; ++j) amax_combine(bv, bi, vals[j], ids[j]);
    block_amax(bv, bi);
    if (threadIdx.x == 0) {
        pv[row * chunks + blockIdx.x] = bv;
        pi[row * chunks + blockIdx.x] = bi;
    }
}

// pass 2: one block per row over `chunks` partials (row stride ld); an all
// -inf / NaN row ends with its lowest index, 0
__global__ __launch_bounds__(256) void k_argmax_final(const float* __restrict__ pv, const uint32_t* __restrict__ pi,
                                                      int64_t chunks, int64_t ld, uint32_t* __restrict__ idx) {
    const int64_t row = blockIdx.x;
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (int64_t c = threadIdx.x; c < chunks; c += blockDim.x) amax_combine(bv, bi, pv[row * ld + c], pi[row * ld + c]);
    block_amax(bv, bi);
    if (threadIdx.x == 0) idx[row] = bi == 0xFFFFFFFFu ? 0u : bi;
}

__global__ void k_fill_u32(uint32_t* p, int64_t n, uint32_t v) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < n) p[t] = v;
}

size_t argmax_workspace_bytes(int64_t m, int64_t n) {
    const int64_t chunks = (n + AMAX_CHUNK - 1) / AMAX_CHUNK;
    return (size_t)(m * chunks) * (sizeof(float) + sizeof(uint32_t));
}

hipError_t launch_argmax(const float* v, int64_t m, int64_t n, uint32_t* idx, void* ws, hipStream_t s) {
    if (m == 0) return hipSuccess;
    if (n == 0) {  // empty rows -> index 0 (a fill kernel: safe under graph capture)
        hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, s, idx, m, 0u);
        return hipGetLastError();
    }
    const int chunks = (int)((n + AMAX_CHUNK - 1) / AMAX_CHUNK);
    float* pv = static_cast<float*>(ws);
    uint32_t* pi = reinterpret_cast<uint32_t*>(pv + m * chunks);
    hipLaunchKernelGGL((k_amax_pass<false>), dim3((unsigned)chunks, (unsigned)m), dim3(256), 0, s, v,
                       (const uint32_t*)nullptr, n, n, chunks, pv, pi);
    hipLaunchKernelGGL(k_argmax_final, dim3((unsigned)m), dim3(256), 0, s, pv, pi, (int64_t)chunks, (int64_t)chunks,
                       idx);
    return hipGetLastError();
}

size_t argmax_partials_tmp_bytes(int64_t m, int64_t nb) { return argmax_workspace_bytes(m, nb); }

// one 1024-thread block per row over all nb partials (independent loads, 8
// per thread per step): one launch where the partials are few
__global__ __launch_bounds__(1024) void k_amax_partials_row(const float* __restrict__ v, const uint32_t* __restrict__ iv,
                                                            int64_t nb, int64_t ld, uint32_t* __restrict__ idx) {
    const int64_t row = blockIdx.x;
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (int64_t c0 = threadIdx.x; c0 < nb; c0 += 1024 * AMAX_PT) {
        float vals[AMAX_PT];
        uint32_t ids[AMAX_PT];
#pragma unroll
        for (int j = 0; j < AMAX_PT; ++j) {
            const int64_t k = c0 + (int64_t)j * 1024;
            const bool in = k < nb;
            vals[j] = in ? v[row * ld + k] : -INFINITY;
            ids[j] = in ? iv[row * ld + k] : 0xFFFFFFFFu;
        }
#pragma unroll
        for (int j = 0; j < AMAX_PT; ++j) amax_combine(bv, bi, vals[j], ids[j]);
    }
    block_amax(bv, bi);
    if (threadIdx.x == 0) idx[row] = bi == 0xFFFFFFFFu ? 0u : bi;
}

// The fused epilogues' partials: a tile whose outputs are all -inf / NaN
// reports (-inf, its first index), so the lowest-index combine still gives
// index 0 for such a row.
hipError_t launch_argmax_partials(const float* v, const uint32_t* i, int64_t m, int64_t nb, int64_t ld,
                                  uint32_t* idx, void* tmp, hipStream_t s) {
    if (m == 0) return hipSuccess;
    if (nb <= 0 || nb > ld) return hipErrorInvalidValue;
    if (nb <= 1024 * AMAX_PT) {
        hipLaunchKernelGGL(k_amax_partials_row, dim3((unsigned)m), dim3(1024), 0, s, v, i, nb, ld, idx);
        return hipGetLastError();
    }
    const int chunks = (int)((nb + AMAX_CHUNK - 1) / AMAX_CHUNK);
    float* pv = static_cast<float*>(tmp);
    uint32_t* pi = reinterpret_cast<uint32_t*>(pv + m * chunks);
    hipLaunchKernelGGL((k_amax_pass<true>), dim3((unsigned)chunks, (unsigned)m), dim3(256), 0, s, v, i, nb, ld, chunks,
                       pv, pi);
    hipLaunchKernelGGL(k_argmax_final, dim3((unsigned)m), dim3(256), 0, s, pv, pi, (int64_t)chunks, (int64_t)chunks,
                       idx);
    return hipGetLastError();
}

}  // namespace thq
