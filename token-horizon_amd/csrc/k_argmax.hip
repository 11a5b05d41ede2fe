// k_argmax.hip — per-row greedy argmax over f32 logits.
//
// Tie rule of engine/src/engine.rs:1891-1898 (greedy_argmax) and candle's
// arg-reduce: a strict '>' scan from (index 0, -inf), so the lowest index
// among equal maxima wins, NaN is never selected and a row of -inf gives 0.
// Two passes: chunks of 4096 elements per block, then one block per row over
// the chunk partials.  The combine (larger value, else lower index) is
// associative, so the result equals the sequential scan's.
#include "thq_dev.hpp"
#include "thq_kernels.hpp"

namespace thq {

constexpr int ARGMAX_CHUNK = 4096;

__device__ __forceinline__ void amax_combine(float& v, uint32_t& i, float v2, uint32_t i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

__device__ __forceinline__ void block_amax(float& v, uint32_t& i) {
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
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

// pass 1: grid (chunks, M)
__global__ __launch_bounds__(256) void k_argmax_chunks(const float* __restrict__ v, int64_t n, int chunks,
                                                       float* __restrict__ pv, uint32_t* __restrict__ pi) {
    const int64_t row = blockIdx.y;
    const int64_t c0 = (int64_t)blockIdx.x * ARGMAX_CHUNK;
    int64_t c1 = c0 + ARGMAX_CHUNK;
    if (c1 > n) c1 = n;
    const float* r = v + row * n;
    float bv = -INFINITY;
    uint32_t bi = 0;
    for (int64_t k = c0 + threadIdx.x; k < c1; k += blockDim.x) {
        const float x = r[k];
        if (x > bv) {
            bv = x;
            bi = (uint32_t)k;
        }
    }
    block_amax(bv, bi);
    if (threadIdx.x == 0) {
        pv[row * chunks + blockIdx.x] = bv;
        pi[row * chunks + blockIdx.x] = bi;
    }
}

// pass 2: one block per row
__global__ __launch_bounds__(256) void k_argmax_final(const float* __restrict__ pv, const uint32_t* __restrict__ pi,
                                                      int chunks, uint32_t* __restrict__ idx) {
    const int64_t row = blockIdx.x;
    float bv = -INFINITY;
    uint32_t bi = 0;
    for (int c = threadIdx.x; c < chunks; c += blockDim.x) amax_combine(bv, bi, pv[row * chunks + c], pi[row * chunks + c]);
    block_amax(bv, bi);
    if (threadIdx.x == 0) idx[row] = bi;
}

__global__ void k_fill_u32(uint32_t* p, int64_t n, uint32_t v) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < n) p[t] = v;
}

size_t argmax_workspace_bytes(int64_t m, int64_t n) {
    const int64_t chunks = (n + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK;
    return (size_t)(m * chunks) * (sizeof(float) + sizeof(uint32_t));
}

hipError_t launch_argmax(const float* v, int64_t m, int64_t n, uint32_t* idx, void* ws, hipStream_t s) {
    if (m == 0) return hipSuccess;
    if (n == 0) {  // empty rows -> index 0 (a fill kernel: safe under graph capture)
        hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, s, idx, m, 0u);
        return hipGetLastError();
    }
    const int chunks = (int)((n + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK);
    float* pv = static_cast<float*>(ws);
    uint32_t* pi = reinterpret_cast<uint32_t*>(pv + m * chunks);
    hipLaunchKernelGGL(k_argmax_chunks, dim3((unsigned)chunks, (unsigned)m), dim3(256), 0, s, v, n, chunks, pv, pi);
    hipLaunchKernelGGL(k_argmax_final, dim3((unsigned)m), dim3(256), 0, s, pv, pi, chunks, idx);
    return hipGetLastError();
}

}  // namespace thq
