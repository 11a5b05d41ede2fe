/*
 * affine_oracle.c — CPU oracle for the engine's MLX affine 4-bit projections.
 *
 * TEST INFRASTRUCTURE ONLY (see thq_oracle.h): the checker the HIP kernels
 * are compared against; the product library never links or calls it.
 *
 * Restates, from the reference tree:
 *   dequant_affine      engine/src/qwen35.rs:110-134
 *   QLin fields / sb    engine/src/qwen35.rs:311-319 (wq U32 [out, in/8],
 *                       sb BF16 [out, 2*ng] = scales | biases per row, as
 *                       Weights::get_lin builds it, qwen35.rs:249-300)
 *   QLin::tiled         engine/src/qwen35.rs:629-697 (addresses q4woff / q4sb,
 *                       engine/src/quant_kernel.rs:1085-1101)
 * and from the crates.io dependency half 2.7.1 (engine/Cargo.lock:1210-1211)
 * its bf16::from_f64 conversion, which dequant_affine rounds with.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "thq_oracle.h"

/* [ext] half 2.7.1 f64_to_bf16: keep the top 32 bits of the f64 (sign,
 * exponent, 20 mantissa bits), then round those 20 bits to bf16's 7 to
 * nearest even.  The 32 low mantissa bits never take part, so a value just
 * above a bf16 tie only by them rounds as the tie.  Overflow -> inf,
 * subnormal results shift in the hidden bit, NaN keeps its top mantissa bits
 * with the quiet bit set. */
uint16_t o_bf16_from_f64_half(double v) {
    uint64_t bits;
    memcpy(&bits, &v, 8);
    const uint32_t x = (uint32_t)(bits >> 32);
    const uint32_t sign = x & 0x80000000u, exp = x & 0x7FF00000u;
    uint32_t man = x & 0x000FFFFFu;
    const uint32_t hs = sign >> 16;
    if (exp == 0x7FF00000u) {
        const uint32_t nan_bit = (man == 0 && (uint32_t)bits == 0) ? 0u : 0x0040u;
        return (uint16_t)(hs | 0x7F80u | nan_bit | (man >> 13));
    }
    const int he = (int)(exp >> 20) - 1023 + 127;
    if (he >= 0xFF) return (uint16_t)(hs | 0x7F80u);
    if (he <= 0) {
        if (14 - he > 21) return (uint16_t)hs;
        man |= 0x00100000u;
        uint32_t hm = man >> (14 - he);
        const uint32_t rb = 1u << (13 - he);
        if ((man & rb) && (man & (3u * rb - 1u))) hm += 1;
        return (uint16_t)(hs | hm);
    }
    const uint32_t r = hs | ((uint32_t)he << 7) | (man >> 13);
    return (uint16_t)(((man & 0x1000u) && (man & 0x2FFFu)) ? r + 1 : r);
}

static inline double bf16_f64(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return (double)f;
}

static inline uint32_t nib(const uint32_t* row, int64_t i) { return (row[i / 8] >> ((i % 8) * 4)) & 0xFu; }

/* dequant_affine with bits = 4: out[o][i] = bf16::from_f64(q * scale + bias)
 * in f64 (a product then a sum, no fusion), g = i / gs. */
void o_affine_dequant_bf16(const uint32_t* wq, const uint16_t* sb, int64_t n, int64_t k, int gs, uint16_t* out) {
    const int64_t ng = k / gs;
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < n; ++o) {
        const uint32_t* wr = wq + o * (k / 8);
        const uint16_t* sr = sb + o * 2 * ng;
        for (int64_t i = 0; i < k; ++i) {
            const int64_t g = i / gs;
            out[o * k + i] = o_bf16_from_f64_half((double)nib(wr, i) * bf16_f64(sr[g]) + bf16_f64(sr[ng + g]));
        }
    }
}

/* the same values rounded once to f32 (the library's f32 dequantization) */
void o_affine_dequant_f32(const uint32_t* wq, const uint16_t* sb, int64_t n, int64_t k, int gs, float* out) {
    const int64_t ng = k / gs;
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < n; ++o) {
        const uint32_t* wr = wq + o * (k / 8);
        const uint16_t* sr = sb + o * 2 * ng;
        for (int64_t i = 0; i < k; ++i) {
            const int64_t g = i / gs;
            out[o * k + i] = (float)((double)nib(wr, i) * bf16_f64(sr[g]) + bf16_f64(sr[ng + g]));
        }
    }
}

/* y[m][o] = sum_i x[m][i] * (q * scale + bias), weights exact, f64 sums */
void o_affine_matmul(const uint32_t* wq, const uint16_t* sb, int64_t n, int64_t k, int gs, const float* x, int64_t m,
                     float* y) {
    const int64_t ng = k / gs;
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < n; ++o) {
        const uint32_t* wr = wq + o * (k / 8);
        const uint16_t* sr = sb + o * 2 * ng;
        for (int64_t r = 0; r < m; ++r) {
            double acc = 0.0;
            for (int64_t i = 0; i < k; ++i) {
                const int64_t g = i / gs;
                acc += (double)x[r * k + i] * ((double)nib(wr, i) * bf16_f64(sr[g]) + bf16_f64(sr[ng + g]));
            }
            y[r * n + o] = (float)acc;
        }
    }
}

/* QLin::tiled (gs = 64): wq_t [tiles][ng][256][8] words, sb_t = scales
 * [(t*ng + g)*256 + col] then biases at + tiles*ng*256; rows past n stay
 * zero (the caller zero-fills both outputs). */
void o_affine_tile(const uint32_t* wq, const uint16_t* sb, int64_t n, int64_t k, uint32_t* wq_t, uint16_t* sb_t) {
    const int64_t ng = k / 64, tiles = (n + 255) / 256;
    const int64_t bias_base = tiles * 256 * ng;
    for (int64_t t = 0; t < tiles; ++t) {
        for (int64_t g = 0; g < ng; ++g) {
            const int64_t rows = n - t * 256 < 256 ? n - t * 256 : 256;
            for (int64_t col = 0; col < rows; ++col) {
                const int64_t row = t * 256 + col;
                memcpy(wq_t + t * ng * 2048 + g * 2048 + col * 8, wq + row * ng * 8 + g * 8, 8 * sizeof(uint32_t));
                sb_t[t * ng * 256 + g * 256 + col] = sb[row * 2 * ng + g];
                sb_t[bias_base + t * ng * 256 + g * 256 + col] = sb[row * 2 * ng + ng + g];
            }
        }
    }
}
