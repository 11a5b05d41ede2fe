// thq_dev.hpp — device-side helpers shared by the gfx950 kernels.
//
// Block formats (GGML, as candle-core's k_quants stores them):
//   Q8_0: 32 weights / 34 B  = f16 d, i8 qs[32]            (repacked on device
//         into 32-row tiles: see q8t_q and q8t_d below)
//   Q4_K: 256 weights / 144 B = f16 d, f16 dmin, u8 scales[12], u8 qs[128]
//         (re-laid on device in row quads, headers re-encoded: see
//         q4k_hdr_from_gguf and q4k_group below)
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

// one v_cvt_pk_bf16_f32 (round to nearest even, like f32_to_bf16)
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef float f32x2_v __attribute__((ext_vector_type(2)));
    const f32x2_v f = {lo, hi};
    const bf16x2_t b = __builtin_convertvector(f, bf16x2_t);
    uint32_t r;
    __builtin_memcpy(&r, &b, 4);
    return r;
}

__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// 16 bytes as an MFMA operand of eight bf16
__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
    bf16x8_t r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

// GGML get_scale_min_k4 on the 12 scale bytes held as three dwords
// s0 = scales[0..3], s1 = scales[4..7], s2 = scales[8..11].
__host__ __device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t& sc,
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

// ---------------------------------------------------------------------------
// On-device Q4_K header.  The 16 header bytes of a GGUF superblock (f16 d,
// f16 dmin, 12 bytes of k4-packed 6-bit scales/mins) are re-encoded at upload
// as four dwords H[p], one per 64-weight part p (sub-blocks 2p and 2p+1):
//   bits  0..5  sc(2p)    bits  6..11 m(2p)
//   bits 12..17 sc(2p+1)  bits 18..23 m(2p+1)
//   bits 24..31 byte p of (d_bits | dmin_bits << 16)
// A lane working on part p decodes its scales from one dword.  Download
// converts back to GGUF bytes.
__host__ __device__ __forceinline__ uint4 q4k_hdr_from_gguf(uint4 g) {
    uint32_t h[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        uint32_t sc0, m0, sc1, m1;
        scale_min_k4(2 * p, g.y, g.z, g.w, sc0, m0);
        scale_min_k4(2 * p + 1, g.y, g.z, g.w, sc1, m1);
        h[p] = sc0 | (m0 << 6) | (sc1 << 12) | (m1 << 18) | (((g.x >> (8 * p)) & 0xFFu) << 24);
    }
    return make_uint4(h[0], h[1], h[2], h[3]);
}

__host__ __device__ __forceinline__ uint4 q4k_hdr_to_gguf(uint4 h) {
    const uint32_t hp[4] = {h.x, h.y, h.z, h.w};
    uint32_t s[3] = {0, 0, 0};
    uint32_t dd = 0;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        dd |= (hp[p] >> 24) << (8 * p);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int j = 2 * p + half;
            const uint32_t sc = (hp[p] >> (12 * half)) & 63u, m = (hp[p] >> (12 * half + 6)) & 63u;
            if (j < 4) {
                s[0] |= sc << (8 * j);
                s[1] |= m << (8 * j);
            } else {
                const int i = j - 4;
                s[2] |= ((sc & 0xFu) | ((m & 0xFu) << 4)) << (8 * i);
                s[0] |= (sc >> 4) << (8 * i + 6);
                s[1] |= (m >> 4) << (8 * i + 6);
            }
        }
    }
    return make_uint4(dd, s[0], s[1], s[2]);
}

// d and dmin of an on-device header
__device__ __forceinline__ float q4k_hdr_d(uint4 h) {
    return f16_to_f32((uint16_t)__builtin_amdgcn_perm(h.y, h.x, 0x0c0c0703u));
}
__device__ __forceinline__ float q4k_hdr_dmin(uint4 h) {
    return f16_to_f32((uint16_t)__builtin_amdgcn_perm(h.w, h.z, 0x0c0c0703u));
}
// (sc, m) of sub-block j
__device__ __forceinline__ void q4k_hdr_sm(uint4 h, int j, uint32_t& sc, uint32_t& m) {
    const uint32_t hp[4] = {h.x, h.y, h.z, h.w};
    const uint32_t w = hp[j >> 1] >> (12 * (j & 1));
    sc = w & 63u;
    m = (w >> 6) & 63u;
}

// MLX affine 4-bit weights (qtype 13 inside the library) share the Q4_K
// row-quad layout below: a 64-weight group is one part p of a 256-weight
// superblock (nibble byte i of the part: low = element i, high = element
// 32 + i), and header dword p holds the group's bf16 scale (low half) and
// bf16 bias (high half); w = scale * q + bias.  Groups of 128 store their
// pair in both 64-halves.
__host__ __device__ __forceinline__ float aff_scale(uint32_t hw) {
    union { uint32_t u; float f; } v = {hw << 16};
    return v.f;
}
__host__ __device__ __forceinline__ float aff_bias(uint32_t hw) {
    union { uint32_t u; float f; } v = {hw & 0xFFFF0000u};
    return v.f;
}

// Q4_K device layout ("row quads").  Rows are grouped by four; group
// g = n/4 occupies nsb*576 bytes (= 4 rows x nsb x 144) at g*nsb*576:
//   nibbles  [r = n%4][h][s][p][16 B]  piece (h, s, p) = bytes 32p+16h .. +15
//                                       of superblock s's 128 nibble bytes
//   headers  [s][p][r][4 B] at +nsb*512 dword p of row r's re-encoded header
// For a K chunk of 16 superblocks, lane 4s+p of a wave reads piece (h, s, p)
// of row r with one 16-B load (the wave reads a contiguous 1 KB) and the four
// rows' header dword p with one more 16-B load.
__host__ __device__ __forceinline__ int64_t q4k_group(int64_t n, int nsb) { return (n >> 2) * (int64_t)nsb * 576; }
__host__ __device__ __forceinline__ int64_t q4k_piece(int64_t n, int nsb, int s, int h, int p) {
    return q4k_group(n, nsb) + (int64_t)(n & 3) * nsb * 128 + (int64_t)h * nsb * 64 + (int64_t)(4 * s + p) * 16;
}
__host__ __device__ __forceinline__ int64_t q4k_hdword(int64_t n, int nsb, int s, int p) {
    return q4k_group(n, nsb) + (int64_t)nsb * 512 + (int64_t)(4 * s + p) * 16 + 4 * (n & 3);
}

// Q4_K / MLX affine tile plane: an optional second copy of a weight
// (thq_weight_add_tiles), 32-row tiles for the 2..8-row decode GEMV.  Record
// (tile t, superblock s) is 4608 contiguous bytes at (t * nsb + s) * 4608:
//   [p][g][n][16 B]  row 32t + n's nibble bytes 32p + 16g .. + 15 of
//                    superblock s (row-quad piece (g, s, p)); 4096 B
//   [n][16 B]        row 32t + n's four on-device header dwords of s; 512 B
// A wave load of part p (64 lanes x 16 B = 1 KB, lane (n, g)) reads whole
// lines and gives each lane its MFMA B-operand piece.  Rows past N are zero.
__host__ __device__ __forceinline__ int64_t q4t_record(int64_t tile, int nsb, int s) {
    return (tile * nsb + s) * 4608;
}
__host__ __device__ __forceinline__ int64_t q4t_bytes(int64_t n, int nsb) { return (n + 31) / 32 * nsb * 4608; }

// Q8_0 device layout, tiles of 32 rows (rows padded to a multiple of 32 with
// zero rows).  nb = K / 32 blocks per row.
//   i8 plane:  [tile][block b][half g][row n][16 B]: row 32t + n's bytes
//              16g .. 16g + 15 of block b.  One block of a tile is 1 KB, so a
//              wave load with lane (n, g) reads it contiguously and each lane
//              gets the MFMA B-operand piece of its row.
//   f16 plane: [tile][chunk c = b / 8][row n][8]: the scales of blocks
//              8c .. 8c + 7 of a row are 16 contiguous bytes (last chunk zero-
//              padded when nb % 8 != 0).
// Offsets: q8t_q in bytes of the i8 plane, q8t_d in f16 units.
__host__ __device__ __forceinline__ int64_t q8t_chunks(int64_t nb) { return (nb + 7) >> 3; }
__host__ __device__ __forceinline__ int64_t q8t_q(int64_t row, int64_t nb, int64_t b, int g) {
    return (((row >> 5) * nb + b) << 10) + ((int64_t)(32 * g + (row & 31)) << 4);
}
__host__ __device__ __forceinline__ int64_t q8t_d(int64_t row, int64_t nb, int64_t b) {
    return (((row >> 5) * q8t_chunks(nb) + (b >> 3)) << 8) + ((row & 31) << 3) + (b & 7);
}
__host__ __device__ __forceinline__ int64_t q8t_q_bytes(int64_t n, int64_t k) { return (n + 31) / 32 * 32 * k; }
__host__ __device__ __forceinline__ int64_t q8t_d_bytes(int64_t n, int64_t k) {
    return (n + 31) / 32 * q8t_chunks(k / 32) * 512;
}

// Streaming loads of weights that a kernel reads exactly once, where one wave
// instruction consumes whole cache lines (the M = 1 GEMVs' 1-KB wave loads):
// the nontemporal hint keeps them from displacing reused data; measured
// 7.1 -> 6.7 us on the 28 MB Q4_K M = 1 GEMV.  Kernels that read a line in
// several instructions (the MFMA decode GEMV's 16-B row pieces) must not use
// it: the line is gone before the next piece and is fetched again (2x slower).
typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream16(const void* p) {
    const u32x4_nt v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Q6_K (GGML type 14, 210 B per 256 weights: u8 ql[128], u8 qh[64], i8
// scales[16], f16 d) on the device: four row-major planes, each starting on a
// 256-B boundary,
//   QL [N][K/2]   QH [N][K/4]   SC [N][K/16] (int8)   D [N][K/256] (f16),
// with the code bits regrouped by 64-weight step j (weights 64j .. 64j+63 of
// the row): step j owns 32 QL bytes at 32j, 16 QH bytes at 16j, 4 scales at
// 4j (GGUF order already groups them so) and d of superblock j/4:
//   code(w) = (QL[32j + w % 32] >> 4 * (w / 32)) & 15
//           | ((QH[16j + w % 16] >> 2 * (w / 16)) & 3) << 4,   w = 0..63
//   weight  = (d * SC[4j + w / 16]) * (code - 32)               (GGML's order)
// so every consumer of a step reads exactly its 52.5 bytes.  In GGUF order
// (GGML dequantize_row_q6_K) step j = 2h + e of half h covers quarters 2e,
// 2e + 1 (32 weights each), whose low nibbles share bytes with the other
// step's and whose high bits share bytes with all four quarters.
struct Q6Layout {
    size_t qh, sc, d, total;
};
__host__ __device__ __forceinline__ Q6Layout q6k_layout(int64_t n, int64_t k) {
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    Q6Layout L;
    size_t o = al((size_t)n * (size_t)k / 2);
    L.qh = o;
    o += al((size_t)n * (size_t)k / 4);
    L.sc = o;
    o += al((size_t)n * (size_t)k / 16);
    L.d = o;
    o += al((size_t)n * (size_t)(k / 256) * 2);
    L.total = o;
    return L;
}

// Last-block tickets (split-K partials, producer epilogues, one-launch
// top-k).  The data another block will read is written and read only with
// agent-scope atomics (16-B or 4-B global stores / loads with sc1), which are
// performed at the level where all XCDs' L2s are coherent, so no cache
// maintenance is needed: every thread that published data calls
// ticket_publish() (s_waitcnt vmcnt(0): its stores have reached that level)
// before the block barrier that precedes ticket_draw(), a relaxed
// device-scope fetch_add; the block that draws the last ticket reads only
// after the ticket has returned (the barrier that shares it).  Release /
// acquire fences would write back and invalidate a whole L2 per block
// (k_gemm_rq split-K: 58.8 against 36.4 us; the M = 5 decoder layer on tile
// planes: 188.6 against 46 us; the 40-row top-32: 84.5 against 27.4 us).
__device__ __forceinline__ void ticket_publish() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ uint32_t ticket_draw(uint32_t* c) {
    return __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
