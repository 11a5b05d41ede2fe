// k_probe.hip — measurement aids for bench.py, built into their own library
// (libthq_probe.so), not into libthq.so: nothing here is part of the product
// ABI.  Each kernel only reads a device buffer once, launched and rotated
// like the decode GEMV it is held against, so the times bound what a single
// launch of that many bytes can reach on this part (a ~28 MB read does not
// reach the sustained HBM rate: ramp-up and drain are part of every launch).
//
//   thqp_hbm_read      grid-stride loop, one 16-B load per lane per iteration
//   thqp_hbm_read_x4   grid-stride loop, four independent 16-B loads per lane
//                      per iteration (more bytes in flight per wave)
//   thqp_gemv_loads    the Q4_K M = 1 GEMV's own load pattern on a row-quad
//                      plane (K <= 4096): 256-thread blocks of four waves, one
//                      row quad per wave, the block's x loads first, then the
//                      wave's nine 1-KB nontemporal loads (headers, then the
//                      eight nibble pieces), x staged in LDS behind a barrier;
//                      no math
//
// Every kernel XORs what it reads and stores only when that XOR equals a
// fixed constant (practically never), so the loads cannot be removed.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef uint32_t u32x4_nt __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ld_nt16(const void* p) {
    const u32x4_nt v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t xor4(uint4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

constexpr uint32_t SINK_KEY = 0x9E3779B9u;

__global__ __launch_bounds__(256) void k_hbm_read(const uint4* __restrict__ p, size_t n16, uint32_t* __restrict__ sink) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    uint32_t acc = 0;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) acc ^= xor4(p[i]);
    if (acc == SINK_KEY) sink[0] = acc;
}

// four loads per lane per iteration, each a whole grid stride apart; the
// tail (fewer than four strides left) takes the one-load loop
__global__ __launch_bounds__(256) void k_hbm_read_x4(const uint4* __restrict__ p, size_t n16, uint32_t* __restrict__ sink) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const uint4 a = p[i], b = p[i + stride], c = p[i + 2 * stride], d = p[i + 3 * stride];
        acc ^= xor4(a) ^ xor4(b) ^ xor4(c) ^ xor4(d);
    }
    for (; i < n16; i += stride) acc ^= xor4(p[i]);
    if (acc == SINK_KEY) sink[0] = acc;
}

// W: row-quad plane of nquads quads of nsb superblocks (576 B each per quad);
// x: K = 256 nsb bf16 values (nsb <= 16)
__global__ __launch_bounds__(256) void k_gemv_loads(const uint8_t* W, const uint16_t* x, int64_t nquads, int nsb,
                                                    uint32_t* __restrict__ sink) {
    __shared__ uint4 lds[512];
    const int lane = threadIdx.x & 63;
    const int64_t gq = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nx = nsb * 32;  // 16-B chunks of x
    const int c0 = threadIdx.x < nx ? threadIdx.x : nx - 1;
    const int c1 = threadIdx.x + 256 < nx ? threadIdx.x + 256 : nx - 1;
    const uint4 xv0 = reinterpret_cast<const uint4*>(x)[c0];
    const uint4 xv1 = reinterpret_cast<const uint4*>(x)[c1];
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    const int64_t q = gq < nquads ? gq : nquads - 1;
    const int li = (lane >> 2) < nsb ? lane : (lane & 3);
    const uint8_t* g = W + q * (int64_t)nsb * 576 + (int64_t)li * 16;
    uint4 v[9];
    v[8] = ld_nt16(g + (int64_t)nsb * 512);
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int h = 0; h < 2; ++h) v[2 * r + h] = ld_nt16(g + (int64_t)r * nsb * 128 + (int64_t)h * nsb * 64);
    lds[threadIdx.x] = xv0;
    lds[threadIdx.x + 256] = xv1;
    __syncthreads();
    uint32_t acc = xor4(lds[(lane * 8) & 511]);
#pragma unroll
    for (int i = 0; i < 9; ++i) acc ^= xor4(v[i]);
    if (gq < nquads && acc == SINK_KEY) sink[0] = acc;
}

}  // namespace

extern "C" {

// 0 on success, else the hipError_t of the launch (or hipErrorInvalidValue)
int thqp_hbm_read(const void* buf, size_t bytes, int blocks, uint32_t* sink, void* stream) {
    if (!buf || !sink || bytes % 16 || ((uintptr_t)buf & 15) || blocks < 1 || blocks > (1 << 20))
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_hbm_read, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4*>(buf), bytes / 16, sink);
    return (int)hipGetLastError();
}

int thqp_hbm_read_x4(const void* buf, size_t bytes, int blocks, uint32_t* sink, void* stream) {
    if (!buf || !sink || bytes % 16 || ((uintptr_t)buf & 15) || blocks < 1 || blocks > (1 << 20))
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_hbm_read_x4, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4*>(buf), bytes / 16, sink);
    return (int)hipGetLastError();
}

// W: nquads * nsb * 576 bytes (16-B aligned); x: 256 * nsb bf16 (16-B aligned)
int thqp_gemv_loads(const void* W, const void* x, int64_t nquads, int nsb, uint32_t* sink, void* stream) {
    if (!W || !x || !sink || nquads < 1 || nsb < 1 || nsb > 16 || ((uintptr_t)W & 15) || ((uintptr_t)x & 15))
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_gemv_loads, dim3((unsigned)((nquads + 3) / 4)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(W),
                       static_cast<const uint16_t*>(x), nquads, nsb, sink);
    return (int)hipGetLastError();
}

}  // extern "C"
