/*
 * baseline.c — the timed CPU baseline: candle's default CPU QMatMul
 * (activations quantized to the weight's VecDotType, integer block dots,
 * f32 block scaling) with AVX2 int8 dot products and OpenMP over output
 * columns, the way [ext] candle-core 0.11.0 k_quants::matmul splits columns
 * over rayon and quantized/avx.rs vectorises vec_dot.
 *
 * TEST INFRASTRUCTURE ONLY (reported beside the GPU number, never the
 * product).  Integer block dots are exact, so results equal the scalar
 * oracle's up to the f32 order of the block-scale accumulation.
 */
#include <immintrin.h>
#include <stdlib.h>
#include <string.h>

#include "thq_oracle.h"
#ifdef _OPENMP
#include <omp.h>
#endif

int o_baseline_has_avx2(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

__attribute__((target("avx2,fma"))) static inline float hsum8(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v), hi = _mm256_extractf128_ps(v, 1);
    lo = _mm_add_ps(lo, hi);
    lo = _mm_add_ps(lo, _mm_movehl_ps(lo, lo));
    lo = _mm_add_ss(lo, _mm_shuffle_ps(lo, lo, 1));
    return _mm_cvtss_f32(lo);
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Q8_0 x Q8_0: |w| (unsigned) times sign-applied x, maddubs -> madd -> f32 */
__attribute__((target("avx2,fma"))) static float dot_q8_0_avx2(int64_t k, const uint8_t* w, const uint8_t* x) {
    __m256 acc = _mm256_setzero_ps();
    const __m256i ones = _mm256_set1_epi16(1);
    for (int64_t b = 0; b < k / OQK8_0; ++b) {
        const uint8_t* wb = w + b * O_Q8_0_BYTES;
        const uint8_t* xb = x + b * O_Q8_0_BYTES;
        __m256i qw = _mm256_loadu_si256((const __m256i*)(wb + 2));
        __m256i qx = _mm256_loadu_si256((const __m256i*)(xb + 2));
        __m256i aw = _mm256_sign_epi8(qw, qw);
        __m256i sx = _mm256_sign_epi8(qx, qw);
        __m256i p16 = _mm256_maddubs_epi16(aw, sx);
        __m256i p32 = _mm256_madd_epi16(p16, ones);
        float d = o_f16_to_f32(rd16(wb)) * o_f16_to_f32(rd16(xb));
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(p32), acc);
    }
    return hsum8(acc);
}

/* Q4_K x Q8_K: nibbles (u8) times q8 (i8) with maddubs, scaled per
 * sub-block by its 6-bit scale through madd, mins through bsums. */
__attribute__((target("avx2,fma"))) static float dot_q4_k_avx2(int64_t k, const uint8_t* w, const uint8_t* x) {
    __m256 acc = _mm256_setzero_ps();
    float acc_m = 0.0f;
    const __m256i m4 = _mm256_set1_epi8(0xF);
    for (int64_t b = 0; b < k / OQK_K; ++b) {
        const uint8_t* wb = w + b * O_Q4_K_BYTES;
        const uint8_t* xb = x + b * O_Q8_K_BYTES;
        float dx;
        memcpy(&dx, xb, 4);
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; ++j) o_get_scale_min_k4(j, wb + 4, &sc[j], &mn[j]);
        int32_t summ = 0;
        const int16_t* bs = (const int16_t*)(xb + 4 + OQK_K);
        for (int j = 0; j < 16; ++j) summ += (int32_t)bs[j] * (int32_t)mn[j / 2];
        const uint8_t* q4 = wb + 16;
        const int8_t* q8 = (const int8_t*)(xb + 4);
        __m256i sumi = _mm256_setzero_si256();
        for (int j = 0; j < 4; ++j) {
            __m256i q = _mm256_loadu_si256((const __m256i*)(q4 + 32 * j));
            __m256i lo = _mm256_and_si256(q, m4);
            __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
            __m256i x0 = _mm256_loadu_si256((const __m256i*)(q8 + 64 * j));
            __m256i x1 = _mm256_loadu_si256((const __m256i*)(q8 + 64 * j + 32));
            __m256i p0 = _mm256_madd_epi16(_mm256_maddubs_epi16(lo, x0), _mm256_set1_epi16(sc[2 * j]));
            __m256i p1 = _mm256_madd_epi16(_mm256_maddubs_epi16(hi, x1), _mm256_set1_epi16(sc[2 * j + 1]));
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p0, p1));
        }
        float d = o_f16_to_f32(rd16(wb)) * dx;
        float dmin = o_f16_to_f32(rd16(wb + 2)) * dx;
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
        acc_m -= dmin * (float)summ;
    }
    return hsum8(acc) + acc_m;
}

int o_baseline_matmul(int type, const uint8_t* w, int64_t n, int64_t k, const float* x, int64_t m, float* y,
                      int threads) {
    if (!o_baseline_has_avx2()) return o_matmul(type, 1, w, n, k, x, m, y, threads);
    int bs = type == O_TYPE_Q8_0 ? OQK8_0 : type == O_TYPE_Q4_K ? OQK_K : 0;
    if (!bs || k % bs) return -1;
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#endif
    size_t rb = o_row_bytes(type, k);
    size_t xrb = type == O_TYPE_Q8_0 ? (size_t)(k / OQK8_0) * O_Q8_0_BYTES : (size_t)(k / OQK_K) * O_Q8_K_BYTES;
    uint8_t* xq = (uint8_t*)malloc(xrb * (size_t)(m > 0 ? m : 1));
    for (int64_t r = 0; r < m; ++r) {
        if (type == O_TYPE_Q8_0) o_quantize_q8_0(x + r * k, xq + r * xrb, k);
        else o_quantize_q8_k(x + r * k, xq + r * xrb, k);
    }
    for (int64_t r = 0; r < m; ++r) {
#pragma omp parallel for schedule(static) num_threads(nt)
        for (int64_t c = 0; c < n; ++c)
            y[r * n + c] = type == O_TYPE_Q8_0 ? dot_q8_0_avx2(k, w + c * rb, xq + r * xrb)
                                               : dot_q4_k_avx2(k, w + c * rb, xq + r * xrb);
    }
    free(xq);
    return 0;
}
